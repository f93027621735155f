// Instances of the fused wave-list scan with fp16 tables for any m % 16 == 0 (m read at run time).
#include "fused_wave.inl"

namespace vk {
WaveScanKernel fused_wave_kernel_hx(int qg, int ng, int ilp, int segments, bool bulk, int threads) {
    return select_wave_kernel<0, true>(qg, ng, ilp, segments, bulk, threads);
}
}  // namespace vk
