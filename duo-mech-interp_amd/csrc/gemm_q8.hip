// Int8 GEMM for the prefill projections: y[m, n] = sum_k x[m, k] W[n, k] s(n, k) for many rows of x (the decode
// step's few rows use gemv.hip). x fp32 [M, K], W int8 [N, K] row-major with one fp32 scale per group of 128 inputs
// of a row (s(n, k) = scale[n][k / 128], the engine's q8 format) or per output row (s(n, k) = scale[n]), y fp32.
//
// Reference: the engine's int8 `matmul` (engine/kernels.js:97-151: 64 x 64 tiles, used when M > 32; q8 weights of
// engine/kernels.js:15-47) and the MLP path with the neuron hook (`swiglu`, engine/kernels_qwen35.js:250-279).
//
// Arithmetic: bf16 MFMA (v_mfma_f32_32x32x16_bf16) with fp32 accumulation. Each x is split into hi = bf16(x) and
// lo = bf16(x - hi), so x = hi + lo up to 2^-17 |x|; the int8 weights are exact in bf16. Two products per tile
// (hi W + lo W) therefore give the fp32 product to about 1e-5 relative, which keeps the prefill on the fp32 numerics
// of the reference path (HF runs these projections in fp32).
//
// Layout: 256 threads = 2 x 2 waves over a BM x 128 output tile (BM 64 or 128), K in steps of 64. Per K step the
// block stages x[BM, 64] (split into hi and lo) and W[128, 64] (int8 -> bf16) in LDS, rows of 64 bf16 = 8 segments of
// 16 bytes, segment s of row r at s ^ (r & 7) (the 32 rows an MFMA operand read touches hit 8 distinct segments).
// The next step's global loads are issued before the current step's MFMAs, so they are in flight during them.
// Blocks run n-fastest inside an m panel: the panel's rows of x stay in L2 while its column tiles pass.
// Group scales (GS): the MFMAs of one group (two K steps) accumulate into a second register set, which is then added
// to the result scaled by the group's scale of the lane's column (one fp32 FMA per accumulator per 128 inputs).
// Epilogues: store, accumulate into y (the residual add after down_proj / out_proj), or SwiGLU over interleaved
// (gate, up) row pairs with the neuron pushes applied, writing y[m, n / 2].
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kGN = 128;  // output columns per block
constexpr int kGK = 64;   // K step

enum GemmEpi : int { kGemmStore = 0, kGemmAccumulate = 1, kGemmSwiglu = 2 };

__device__ __forceinline__ int gsw(int r, int s) { return s ^ (r & 7); }
__device__ __forceinline__ float gemm_silu(float x) { return x / (1.f + __expf(-x)); }

__device__ __forceinline__ float gemm_push(const q35_push* ps, int n, int row, float a) {
  const int pn = ps->neuron;
  if (pn != n && pn >= 0) return a;
  const float v = ps->vals[row];
  return ps->mode ? a * v : a + v;
}

// 8 consecutive fp32 values as bf16 hi and lo parts
__device__ __forceinline__ void split8(const f32x4& a, const f32x4& b, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = e < 4 ? a[e] : b[e - 4];
    const __bf16 h = (__bf16)x;
    hi[e] = h;
    lo[e] = (__bf16)(x - (float)h);
  }
}
// 8 int8 values (two 32-bit words) as bf16 (exact)
__device__ __forceinline__ bf16x8 i8tobf(uint32_t w0, uint32_t w1) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t w = e < 4 ? w0 : w1;
    r[e] = (__bf16)(float)((int32_t)(w << (24 - 8 * (e & 3))) >> 24);
  }
  return r;
}

template <int BM, int EPI, bool GS>
__global__ __launch_bounds__(256, 2) void gemm_q8_kernel(const float* __restrict__ X, int64_t ldx,
                                                         const int8_t* __restrict__ W, const float* __restrict__ ws,
                                                         float* __restrict__ Y, int64_t ldy, int M, int N, int K,
                                                         const q35_push* __restrict__ pushes, int npush, int T) {
  static_assert(BM == 64 || BM == 128, "rows per block");
  constexpr int MT = BM / 64;         // 32-row MFMA tiles per wave along M (a wave covers BM / 2 rows)
  constexpr int TPR = 256 / BM;       // threads per staged row of x
  constexpr int SPT = 8 / TPR;        // 16-byte segments (8 k values) of x per thread
  __shared__ __attribute__((aligned(16))) bf16x8 Ah[BM * 8];
  __shared__ __attribute__((aligned(16))) bf16x8 Al[BM * 8];
  __shared__ __attribute__((aligned(16))) bf16x8 Bs[kGN * 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int nbn = (N + kGN - 1) / kGN;
  const int bm = blockIdx.x / nbn, bn = blockIdx.x - bm * nbn;
  const int m0 = bm * BM, n0 = bn * kGN;

  // staging assignment: x row ar, segments as0 .. as0 + SPT - 1; W row br, segments 4 bh .. 4 bh + 3
  const int ar = tid / TPR, as0 = (tid % TPR) * SPT;
  const int br = tid >> 1, bh = tid & 1;
  const bool av = m0 + ar < M, bv = n0 + br < N;
  const float* xrow = X + (size_t)min(m0 + ar, M - 1) * ldx + 8 * as0;
  const int8_t* wrow = W + (size_t)min(n0 + br, N - 1) * K + 32 * bh;

  f32x4 xa[SPT][2];
  u32x4 wb[2];
  auto load = [&](int k0) {
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      xa[s][0] = *reinterpret_cast<const f32x4*>(xrow + k0 + 8 * s);
      xa[s][1] = *reinterpret_cast<const f32x4*>(xrow + k0 + 8 * s + 4);
    }
    wb[0] = *reinterpret_cast<const u32x4*>(wrow + k0);
    wb[1] = *reinterpret_cast<const u32x4*>(wrow + k0 + 16);
  };
  auto stage = [&]() {
    const bf16x8 z = {};
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      bf16x8 hi, lo;
      split8(xa[s][0], xa[s][1], hi, lo);
      const int idx = ar * 8 + gsw(ar, as0 + s);
      Ah[idx] = av ? hi : z;
      Al[idx] = av ? lo : z;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4& w = wb[j >> 1];
      const bf16x8 b = i8tobf(w[2 * (j & 1)], w[2 * (j & 1) + 1]);
      Bs[br * 8 + gsw(br, 4 * bh + j)] = bv ? b : z;
    }
  };

  f32x16 acc[MT][2], gacc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      acc[mt][nt] = zero16();
      gacc[mt][nt] = zero16();
    }

  const int l32 = lane & 31, lh = lane >> 5;
  // GS: the lane's two columns' scale rows (column n = n0 + wn 64 + 32 nt + l32)
  const float* srow[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) srow[nt] = ws + (size_t)min(n0 + wn * 64 + 32 * nt + l32, N - 1) * (K >> 7);
  float gsc[2] = {0.f, 0.f};
  load(0);
  for (int k0 = 0; k0 < K; k0 += kGK) {
    __syncthreads();  // every wave is done reading the previous step's tiles
    stage();
    if (k0 + kGK < K) load(k0 + kGK);  // next step's loads fly during this step's MFMAs
    if (GS && (k0 & 127) == 0) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) gsc[nt] = srow[nt][k0 >> 7];
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int sg = 2 * kk + lh;
      bf16x8 ah[MT], al[MT], b[2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int r = wm * (BM / 2) + 32 * mt + l32;
        ah[mt] = Ah[r * 8 + gsw(r, sg)];
        al[mt] = Al[r * 8 + gsw(r, sg)];
      }
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int r = wn * 64 + 32 * nt + l32;
        b[nt] = Bs[r * 8 + gsw(r, sg)];
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          f32x16& d = GS ? gacc[mt][nt] : acc[mt][nt];
          d = mfma32(ah[mt], b[nt], d);
          d = mfma32(al[mt], b[nt], d);
        }
    }
    if (GS && ((k0 + kGK) & 127) == 0) {  // end of a group: fold it in with its scale
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[mt][nt][r] += gsc[nt] * gacc[mt][nt][r];
          gacc[mt][nt] = zero16();
        }
    }
  }

  // epilogue: lane holds column n = n0 + wn 64 + 32 nt + l32, rows m0 + wm BM/2 + 32 mt + 8 (r / 4) + 4 lh + r % 4
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int n = n0 + wn * 64 + 32 * nt + l32;
    const float s = GS ? 1.f : ws[min(n, N - 1)];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * (BM / 2) + 32 * mt + 8 * (r >> 2) + 4 * lh + (r & 3);
        const float v = acc[mt][nt][r] * s;
        if (EPI == kGemmSwiglu) {
          const float up = __shfl_xor(v, 1, 64);  // the odd column of the pair sits in the neighbouring lane
          if ((l32 & 1) == 0 && m < M && n + 1 < N) {
            const int neuron = n >> 1, row = min(m / T, 3);
            float a = gemm_silu(v) * up;
            for (int p = 0; p < npush; ++p) a = gemm_push(pushes + p, neuron, row, a);
            Y[(size_t)m * ldy + neuron] = a;
          }
        } else if (m < M && n < N) {
          float* dst = Y + (size_t)m * ldy + n;
          *dst = EPI == kGemmAccumulate ? *dst + v : v;
        }
      }
    }
  }
}

}  // namespace q35

extern "C" int q35_gemm_q8(const float* x, int64_t ldx, const int8_t* W, int w_dtype, const float* w_scale,
                           float* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue,
                           const q35_push* pushes, int64_t npush, int64_t T, q35_stream_t stream) {
  using namespace q35;
  if (!x || !W || !w_scale || !y || M <= 0 || N <= 0 || K <= 0 || T <= 0) return Q35_EINVAL;
  if (w_dtype != Q35_I8 && w_dtype != Q35_I8_G128) return Q35_EUNSUPPORTED;
  const bool gs = w_dtype == Q35_I8_G128;
  if (gs && K % 128 != 0) return Q35_EUNSUPPORTED;
  if (epilogue < kGemmStore || epilogue > kGemmSwiglu) return Q35_EINVAL;
  if (npush < 0 || (npush > 0 && !pushes) || npush > 64) return Q35_EINVAL;
  if (epilogue == kGemmSwiglu ? (N % 2 != 0 || ldy < N / 2) : ldy < N) return Q35_EINVAL;
  if (ldx < K) return Q35_EINVAL;
  if (K % kGK != 0 || ldx % 4 != 0 || ((uintptr_t)x & 15) || ((uintptr_t)W & 15)) return Q35_EUNSUPPORTED;
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return Q35_EUNSUPPORTED;
  const int64_t nbn = (N + kGN - 1) / kGN;
  // 128-row tiles when they still give at least two blocks per compute unit, else 64-row tiles
  const bool big = ((M + 127) / 128) * nbn >= 512;
  const int BM = big ? 128 : 64;
  const int64_t nblocks = ((M + BM - 1) / BM) * nbn;
  if (nblocks > 0x7fffffff) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define Q35_GEMM_LAUNCH(BMV, E, G)                                                                               \
  hipLaunchKernelGGL((gemm_q8_kernel<BMV, E, G>), dim3((unsigned)nblocks), dim3(256), 0, st, x, ldx, W, w_scale, \
                     y, ldy, (int)M, (int)N, (int)K, pushes, (int)npush, (int)T)
#define Q35_GEMM_EPI(BMV, G)                                              \
  if (epilogue == kGemmStore) Q35_GEMM_LAUNCH(BMV, kGemmStore, G);        \
  else if (epilogue == kGemmAccumulate) Q35_GEMM_LAUNCH(BMV, kGemmAccumulate, G); \
  else Q35_GEMM_LAUNCH(BMV, kGemmSwiglu, G);
  if (big) {
    if (gs) { Q35_GEMM_EPI(128, true) } else { Q35_GEMM_EPI(128, false) }
  } else {
    if (gs) { Q35_GEMM_EPI(64, true) } else { Q35_GEMM_EPI(64, false) }
  }
#undef Q35_GEMM_EPI
#undef Q35_GEMM_LAUNCH
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
