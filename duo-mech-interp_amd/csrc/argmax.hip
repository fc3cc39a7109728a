// Per-row argmax over the last dimension (greedy sampling of the decode step): the engine's WGSL `argmax`
// (engine/kernels.js:260-283, one workgroup per row, strict > while scanning so the lowest index wins within a
// thread, and the lower index on equal values when two candidates meet), which is also torch.argmax's tie rule.
//
// One block of 1024 threads per row: thread t scans 4 consecutive elements at a time (16-byte loads, 8 in flight per
// round), then the (value, index) pairs are reduced across the wave with DPP-free shuffles and across the 16 waves in
// LDS. Bandwidth bound on one CU per row (a 151936-wide fp32 row is 0.6 MB); the decode step has a few rows.
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

__device__ __forceinline__ void amax_take(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float* __restrict__ x, int64_t ldx, int n,
                                                           int32_t* __restrict__ idx, float* __restrict__ val) {
  Q35_ARGS_UPFRONT(x, ldx, n, idx, val);
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* xr = x + (int64_t)row * ldx;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  // elements [h0, h0 + nv) are 16-byte aligned and read four at a time; the few before and after one at a time
  const int h0 = min((int)((4 - (((uintptr_t)xr >> 2) & 3)) & 3), n);
  const int nv = (n - h0) & ~3;
  constexpr int U = 8;
  for (int base = h0 + 4 * tid; base < h0 + nv; base += 4 * 1024 * U) {
    f32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = min(base + 4 * 1024 * u, h0 + nv - 4);
      r[u] = *reinterpret_cast<const f32x4*>(xr + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + 4 * 1024 * u;
      if (i < h0 + nv) {
#pragma unroll
        for (int e = 0; e < 4; ++e) amax_take(bv, bi, r[u][e], i + e);
      }
    }
  }
  if (tid < h0) amax_take(bv, bi, xr[tid], tid);
  for (int i = h0 + nv + tid; i < n; i += 1024) amax_take(bv, bi, xr[i], i);
  // -inf everywhere (or an empty row) still reports index 0, as a scan from -inf with strict > would not: the WGSL
  // kernel starts from -3.4e38 and index 0
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    amax_take(bv, bi, ov, oi);
  }
  __shared__ float sv[16];
  __shared__ int si[16];
  if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
  __syncthreads();
  if (tid == 0) {
    float v = sv[0];
    int i = si[0];
    for (int w = 1; w < 16; ++w) amax_take(v, i, sv[w], si[w]);
    if (i == 0x7fffffff) i = 0;
    idx[row] = i;
    if (val) val[row] = v;
  }
}

}  // namespace q35

extern "C" int q35_argmax_rows(const float* x, int64_t ldx, int64_t rows, int64_t n, int32_t* idx, float* val,
                               q35_stream_t stream) {
  using namespace q35;
  if (!x || !idx || rows <= 0 || n <= 0 || ldx < n) return Q35_EINVAL;
  if (rows > 0x7fffffff || n > 0x7fffffff - 4 * 1024 * 8 || ((uintptr_t)x & 3)) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)rows), dim3(1024), 0, st, x, ldx, (int)n, idx, val);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
