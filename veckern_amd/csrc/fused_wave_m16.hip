// Instances of the fused wave-list scan for m = 16.
#include "fused_wave.inl"

namespace vk {
WaveScanKernel fused_wave_kernel_m16(int qg, int ng, int ilp, int segments, bool bulk, int threads) {
    return select_wave_kernel<16, false>(qg, ng, ilp, segments, bulk, threads);
}
}  // namespace vk
