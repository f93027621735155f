// Inverted-list (IVF) instances of the fused wave-list scan for m = 32.
#include "fused_wave.inl"

namespace vk {
WaveScanKernel ivf_kernel_m32(int segments) { return select_ivf_kernel<32>(segments); }
}  // namespace vk
