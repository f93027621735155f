// Inverted-list (IVF) instances of the fused wave-list scan for any m % 16 == 0 (m read at run time).
#include "fused_wave.inl"

namespace vk {
WaveScanKernel ivf_kernel_mx(int segments) { return select_ivf_kernel<0>(segments); }
}  // namespace vk
