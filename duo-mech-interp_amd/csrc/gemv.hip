// Small-M matrix-vector products for the decode step: y[m, n] = s[n] * sum_k x[m, k] W[n, k] for M <= 8 rows of x,
// W row-major [N, K] in int8 with one fp32 scale per output row (the int8 per-output-channel MLP weights), or fp32
// (scale 1). HBM-bound on W: every weight byte is read once.
//
// Reference: the engine's int8 `matvec` (engine/kernels.js:57-90; it quantizes per group of 128 inputs, this build
// per output channel) and its MLP path with the neuron hook (`swiglu`, engine/kernels_qwen35.js:250-279: a[m, n] =
// silu(gate) * up, then for each push of the layer whose neuron is n or every neuron, add or multiply by the push's
// value for the row; the row index is clamped to 3).
//
// Layout: a block of 4 waves takes 16 output rows; lane l works on row l / 4 and, per 64-input step (int8; 16 for
// fp32), the 16 bytes at l % 4, so a wave load covers 16 rows x 64 contiguous bytes. The four waves split K in
// quarters; x (M x K fp32) is staged in LDS once per block and read as broadcasts. Per-row sums: two DPP steps across
// the 4 lanes of a row, then across the 4 waves in LDS. Epilogues: store, accumulate into y (the residual add after
// down_proj), or SwiGLU over interleaved (gate, up) row pairs with the neuron pushes applied (gate_up_proj).
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

enum GemvEpi : int { kEpiStore = 0, kEpiAccumulate = 1, kEpiSwiglu = 2 };

__device__ __forceinline__ float gsilu(float x) { return x / (1.f + __expf(-x)); }

// one push applied to activation a of neuron n (fields read straight from the record: no copy of the value array)
__device__ __forceinline__ float apply_push(const q35_push* ps, int n, int row, float a) {
  const int pn = ps->neuron;
  if (pn != n && pn >= 0) return a;
  const float v = ps->vals[row];
  return ps->mode ? a * v : a + v;
}

template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// 16 bytes of weights as fp32: int8 x 16 or fp32 x 4
template <typename TW> struct WChunk;
template <> struct WChunk<int8_t> {
  static constexpr int kElems = 16;
  u32x4 r;
  __device__ __forceinline__ void load(const int8_t* p) { r = *reinterpret_cast<const u32x4*>(p); }
  __device__ __forceinline__ float at(int i) const {
    const uint32_t w = r[i >> 2];
    return (float)(int)((int32_t)(w << (24 - 8 * (i & 3))) >> 24);
  }
};
template <> struct WChunk<float> {
  static constexpr int kElems = 4;
  f32x4 r;
  __device__ __forceinline__ void load(const float* p) { r = *reinterpret_cast<const f32x4*>(p); }
  __device__ __forceinline__ float at(int i) const { return r[i]; }
};

template <typename TW, int MP, int EPI, int U>
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x, int64_t ldx, const TW* __restrict__ W,
                                                   const float* __restrict__ wscale, float* __restrict__ y,
                                                   int64_t ldy, int M, int N, int K,
                                                   const q35_push* __restrict__ pushes, int npush, int T) {
  constexpr int E = WChunk<TW>::kElems;  // weights per lane per 16-byte load
  constexpr int STEP = 4 * E;            // inputs per step of a row (4 lanes)
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [MP][K]
  __shared__ float red[4][16][MP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane >> 2, qd = lane & 3;
  const int n = blockIdx.x * 16 + r;
  const TW* wrow = W + (size_t)min(n, N - 1) * K;
  const int kq = K / 4, kb = wave * kq;
  // U steps (U 16-byte loads per lane) in flight per iteration; the first iteration's weight loads are issued before
  // x is staged, so that their latency covers the staging
  WChunk<TW> wc[U];
  auto issue = [&](int k0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = min(k0 + u * STEP, kb + kq - STEP) + qd * E;
      wc[u].load(wrow + k);
    }
  };
  issue(kb);
  asm volatile("" ::: "memory");
  for (int i = tid; i < MP * K / 4; i += 256) {
    const int m = (4 * i) / K, k = 4 * i - m * K;
    f32x4 v = zero4();
    if (m < M) v = *reinterpret_cast<const f32x4*>(x + m * ldx + k);
    *reinterpret_cast<f32x4*>(xs + m * K + k) = v;
  }
  __syncthreads();
  float acc[MP];
#pragma unroll
  for (int m = 0; m < MP; ++m) acc[m] = 0.f;
  for (int k0 = kb; k0 < kb + kq; k0 += U * STEP) {
    if (k0 != kb) issue(k0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k0 + u * STEP >= kb + kq) break;
      const int k = k0 + u * STEP + qd * E;
#pragma unroll
      for (int m = 0; m < MP; ++m) {
        const float* xr = xs + m * K + k;
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < E; c += 4) {
          const f32x4 xv = *reinterpret_cast<const f32x4*>(xr + c);
#pragma unroll
          for (int e = 0; e < 4; ++e) s += wc[u].at(c + e) * xv[e];
        }
        acc[m] += s;
      }
    }
  }
  // the 4 lanes of a row (a quad): quad_perm [1,0,3,2] then [2,3,0,1]
#pragma unroll
  for (int m = 0; m < MP; ++m) {
    acc[m] += dpp_f<0xB1>(acc[m]);
    acc[m] += dpp_f<0x4E>(acc[m]);
  }
  if (qd == 0) {
#pragma unroll
    for (int m = 0; m < MP; ++m) red[wave][r][m] = acc[m];
  }
  __syncthreads();
  if (EPI != kEpiSwiglu) {
    if (tid < 16 * MP) {
      const int rr = tid / MP, m = tid - rr * MP;
      const int nn = blockIdx.x * 16 + rr;
      if (m < M && nn < N) {
        float v = red[0][rr][m] + red[1][rr][m] + red[2][rr][m] + red[3][rr][m];
        if (wscale) v *= wscale[nn];
        float* dst = y + m * ldy + nn;
        *dst = EPI == kEpiAccumulate ? *dst + v : v;
      }
    }
  } else {
    // rows 2 j and 2 j + 1 of the block are gate and up of neuron blockIdx.x * 8 + j
    if (tid < 8 * MP) {
      const int j = tid / MP, m = tid - j * MP;
      const int ng = blockIdx.x * 16 + 2 * j;
      const int neuron = ng >> 1;
      if (m < M && ng + 1 < N) {
        float g = red[0][2 * j][m] + red[1][2 * j][m] + red[2][2 * j][m] + red[3][2 * j][m];
        float u = red[0][2 * j + 1][m] + red[1][2 * j + 1][m] + red[2][2 * j + 1][m] + red[3][2 * j + 1][m];
        if (wscale) { g *= wscale[ng]; u *= wscale[ng + 1]; }
        float a = gsilu(g) * u;
        const int row = min(m / T, 3);
        for (int p = 0; p < npush; ++p) a = apply_push(pushes + p, neuron, row, a);
        y[m * ldy + neuron] = a;
      }
    }
  }
}

// a[m, n] = silu(gu[m, n]) * gu[m, I + n] with the pushes applied (the prefill form over a [gate | up] projection)
__global__ __launch_bounds__(256) void swiglu_push_kernel(const float* __restrict__ gu, float* __restrict__ a,
                                                          int64_t M, int I, const q35_push* __restrict__ pushes,
                                                          int npush, int T) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * I) return;
  const int64_t m = i / I;
  const int n = (int)(i - m * I);
  float v = gsilu(gu[m * 2 * I + n]) * gu[m * 2 * I + I + n];
  const int row = (int)min(m / T, (int64_t)3);
  for (int p = 0; p < npush; ++p) v = apply_push(pushes + p, n, row, v);
  a[i] = v;
}

}  // namespace q35

namespace {
template <typename TW, int EPI, int U>
void gemv_launch_u(const float* x, int64_t ldx, const TW* W, const float* wscale, float* y, int64_t ldy, int64_t M,
                   int64_t N, int64_t K, const q35_push* pushes, int npush, int64_t T, hipStream_t st) {
  using namespace q35;
  const int mp = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const size_t lds = (size_t)mp * K * sizeof(float);
  const dim3 grid((unsigned)((N + 15) / 16)), block(256);
#define Q35_GEMV(MP)                                                                                                  \
  hipLaunchKernelGGL((gemv_kernel<TW, MP, EPI, U>), grid, block, lds, st, x, ldx, W, wscale, y, ldy, (int)M,      \
                     (int)N, (int)K, pushes, npush, (int)T)
  switch (mp) {
    case 1: Q35_GEMV(1); break;
    case 2: Q35_GEMV(2); break;
    case 4: Q35_GEMV(4); break;
    default: Q35_GEMV(8); break;
  }
#undef Q35_GEMV
}

// steps of a wave's K quarter: all in flight at once up to 16
template <typename TW, int EPI>
int gemv_launch(const float* x, int64_t ldx, const TW* W, const float* wscale, float* y, int64_t ldy, int64_t M,
                int64_t N, int64_t K, const q35_push* pushes, int npush, int64_t T, hipStream_t st) {
  using namespace q35;
  const int64_t steps = K / 4 / (4 * WChunk<TW>::kElems);
  if (steps <= 4)
    gemv_launch_u<TW, EPI, 4>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, st);
  else if (steps <= 8)
    gemv_launch_u<TW, EPI, 8>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, st);
  else
    gemv_launch_u<TW, EPI, 16>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, st);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
}  // namespace

extern "C" int q35_gemv(const float* x, int64_t ldx, const void* W, int w_dtype, const float* w_scale, float* y,
                        int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes,
                        int64_t npush, int64_t T, q35_stream_t stream) {
  using namespace q35;
  if (!x || !W || !y || M <= 0 || N <= 0 || K <= 0 || ldx < K || T <= 0) return Q35_EINVAL;
  if (npush < 0 || (npush > 0 && !pushes)) return Q35_EINVAL;
  if (epilogue == kEpiSwiglu ? (N & 1) || ldy < N / 2 : ldy < N) return Q35_EINVAL;
  if (epilogue != kEpiStore && epilogue != kEpiAccumulate && epilogue != kEpiSwiglu) return Q35_EINVAL;
  if (w_dtype != Q35_I8 && w_dtype != Q35_F32) return Q35_EUNSUPPORTED;
  if (M > 8 || (K % 256) != 0 || (ldx & 3) || ((uintptr_t)x & 15) || ((uintptr_t)W & 15)) return Q35_EUNSUPPORTED;
  const int mp = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  if ((int64_t)mp * K * 4 > 64 * 1024 || N > 0x7fffffff || npush > 64) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int np = (int)npush;
  if (w_dtype == Q35_I8) {
    if (epilogue == kEpiStore) return gemv_launch<int8_t, kEpiStore>(x, ldx, (const int8_t*)W, w_scale, y, ldy, M, N, K, pushes, np, T, st);
    if (epilogue == kEpiAccumulate) return gemv_launch<int8_t, kEpiAccumulate>(x, ldx, (const int8_t*)W, w_scale, y, ldy, M, N, K, pushes, np, T, st);
    return gemv_launch<int8_t, kEpiSwiglu>(x, ldx, (const int8_t*)W, w_scale, y, ldy, M, N, K, pushes, np, T, st);
  }
  if (epilogue == kEpiStore) return gemv_launch<float, kEpiStore>(x, ldx, (const float*)W, w_scale, y, ldy, M, N, K, pushes, np, T, st);
  if (epilogue == kEpiAccumulate) return gemv_launch<float, kEpiAccumulate>(x, ldx, (const float*)W, w_scale, y, ldy, M, N, K, pushes, np, T, st);
  return gemv_launch<float, kEpiSwiglu>(x, ldx, (const float*)W, w_scale, y, ldy, M, N, K, pushes, np, T, st);
}

extern "C" int q35_swiglu_push(const float* gu, float* a, int64_t M, int64_t I, const q35_push* pushes,
                               int64_t npush, int64_t T, q35_stream_t stream) {
  using namespace q35;
  if (!gu || !a || M <= 0 || I <= 0 || T <= 0 || npush < 0 || (npush > 0 && !pushes)) return Q35_EINVAL;
  if (M * I > ((int64_t)1 << 40) || (M * I + 255) / 256 > 0x7fffffff || npush > 64 || I > 0x7fffffff)
    return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(swiglu_push_kernel, dim3((unsigned)((M * I + 255) / 256)), dim3(256), 0, st, gu, a, M, (int)I,
                     pushes, (int)npush, (int)T);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
