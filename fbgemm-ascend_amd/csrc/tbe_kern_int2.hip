// tbe_kern_int2.hip — pooled TBE kernels for INT2 rows (per-bag and
// row-stream variants); compiled separately so the library builds in parallel.
#include "tbe_kernels.h"

namespace tbe {
template KernelFn fast_kernel_lg<TBE_TY_INT2>(int, bool, bool, bool);
template KernelFn fast_kernel_a64_lg<TBE_TY_INT2>(int, bool, bool);
template KernelFn stream_kernel_lg<TBE_TY_INT2>(int, bool, bool);
template KernelFn nobag_kernel_lg<TBE_TY_INT2>(int, bool, bool);
}  // namespace tbe
