// Inverted-list (IVF) instances of the fused wave-list scan for m = 64.
#include "fused_wave.inl"

namespace vk {
WaveScanKernel ivf_kernel_m64(int segments) { return select_ivf_kernel<64>(segments); }
}  // namespace vk
