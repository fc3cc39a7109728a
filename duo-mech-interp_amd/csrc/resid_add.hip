// Residual steering add: x[r, t, :] += vecs[row_vec(r), :] at every position (prefill and decode alike).
// Semantics: tests/engine_ref.py:49-53 (forward hook on layers[12] adding s * vec to the layer output) and the WGSL
// `resAdd` (engine/kernels.js:190-203). HBM-bound elementwise pass: 16-byte vector loads/stores along H.
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

template <typename T>
__global__ __launch_bounds__(256) void resid_add_rows_kernel(T* __restrict__ x, const float* __restrict__ vecs,
                                                             const int32_t* __restrict__ vec_of_row, int64_t rows,
                                                             int64_t Tlen, int H, int nvec) {
  Q35_ARGS_UPFRONT(x, vecs, vec_of_row, rows, Tlen, H, nvec);
  // one block per (row, position); 4 elements per thread per step
  const int64_t m = blockIdx.x;  // flattened (row, position)
  const int64_t r = m / Tlen;
  const int vi = vec_of_row ? vec_of_row[r] : (int)(r < nvec - 1 ? r : nvec - 1);
  if (vi < 0 || vi >= nvec) return;
  T* xr = x + m * (int64_t)H;
  const float* vr = vecs + (int64_t)vi * H;
  for (int i = threadIdx.x * 4; i < H; i += blockDim.x * 4) {
    if (i + 3 < H) {
#pragma unroll
      for (int c = 0; c < 4; ++c) xr[i + c] = from_f32<T>(to_f32(xr[i + c]) + vr[i + c]);
    } else {
      for (int c = 0; i + c < H; ++c) xr[i + c] = from_f32<T>(to_f32(xr[i + c]) + vr[i + c]);
    }
  }
}

}  // namespace q35

extern "C" int q35_resid_add_rows(void* x, const float* vecs, const int32_t* vec_of_row, int64_t rows, int64_t T,
                                  int64_t H, int64_t nvec, int dtype, q35_stream_t stream) {
  using namespace q35;
  if (!x || !vecs || rows <= 0 || T <= 0 || H <= 0 || nvec <= 0) return Q35_EINVAL;
  if (H > (1 << 20) || rows * T > (int64_t)0x7fffffff) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((unsigned)(rows * T)), block(256);
  if (dtype == Q35_F32)
    hipLaunchKernelGGL(resid_add_rows_kernel<float>, grid, block, 0, st, (float*)x, vecs, vec_of_row, rows, T,
                       (int)H, (int)nvec);
  else if (dtype == Q35_BF16)
    hipLaunchKernelGGL(resid_add_rows_kernel<__bf16>, grid, block, 0, st, (__bf16*)x, vecs, vec_of_row, rows, T,
                       (int)H, (int)nvec);
  else
    return Q35_EUNSUPPORTED;
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
