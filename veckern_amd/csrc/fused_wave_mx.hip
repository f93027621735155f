// Instances of the fused wave-list scan for any m % 16 == 0 (m read at run time).
#include "fused_wave.inl"

namespace vk {
WaveScanKernel fused_wave_kernel_mx(int qg, int ng, int ilp, int segments, bool bulk, int threads) {
    return select_wave_kernel<0, false>(qg, ng, ilp, segments, bulk, threads);
}
}  // namespace vk
