// Inverted-list (IVF) instances of the fused wave-list scan for m = 16.
#include "fused_wave.inl"

namespace vk {
WaveScanKernel ivf_kernel_m16(int segments) { return select_ivf_kernel<16>(segments); }
}  // namespace vk
