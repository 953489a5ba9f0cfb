// Linear map of a few rows for decode steps (gfx950): the launch of
// rows_detail::linear_rows_block (linear_rows_body.h, which describes it).

#include "linear_rows_body.h"

namespace kch {

namespace {

template <typename T, typename WT>
__global__ __launch_bounds__(256) void linear_rows_kernel(LinearRowsParams p) {
  rows_detail::linear_rows_block<T, WT>(p, (int)blockIdx.x);
}

}  // namespace

template <typename T>
static void linear_rows_launch(const LinearRowsParams& p, hipStream_t s) {
  const dim3 grid((unsigned)((p.N + 15) / 16)), block(256);
  if (!p.ln_w) {
    hipLaunchKernelGGL((linear_rows_kernel<T, void>), grid, block, 0, s, p);
    return;
  }
  const size_t lds = (size_t)p.M * (p.K + 8) * sizeof(T);
  if (p.ln_wdtype == DT_F32) hipLaunchKernelGGL((linear_rows_kernel<T, float>), grid, block, lds, s, p);
  else if (p.ln_wdtype == DT_BF16) hipLaunchKernelGGL((linear_rows_kernel<T, bf16_t>), grid, block, lds, s, p);
  else hipLaunchKernelGGL((linear_rows_kernel<T, _Float16>), grid, block, lds, s, p);
}

hipError_t linear_rows_dispatch(const LinearRowsParams& p, int dtype, hipStream_t s) {
  if (dtype == DT_BF16) linear_rows_launch<bf16_t>(p, s);
  else linear_rows_launch<_Float16>(p, s);
  return hipGetLastError();
}

}  // namespace kch
