// Instances of the fused wave-list scan for m = 64.
#include "fused_wave.inl"

namespace vk {
WaveScanKernel fused_wave_kernel_m64(int qg, int ng, int ilp, int segments, bool bulk, int threads) {
    return select_wave_kernel<64, false>(qg, ng, ilp, segments, bulk, threads);
}
}  // namespace vk
