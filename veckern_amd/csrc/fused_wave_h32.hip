// Instances of the fused wave-list scan with fp16 tables for m = 32.
#include "fused_wave.inl"

namespace vk {
WaveScanKernel fused_wave_kernel_h32(int qg, int ng, int ilp, int segments, bool bulk, int threads) {
    return select_wave_kernel<32, true>(qg, ng, ilp, segments, bulk, threads);
}
}  // namespace vk
