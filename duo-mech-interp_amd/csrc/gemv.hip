// Small-M matrix-vector products for the decode step: y[m, n] = sum_k x[m, k] W[n, k] s(n, k) for M <= 8 rows of x,
// W row-major [N, K] in int8 with one fp32 scale per group of 128 inputs of a row (s(n, k) = scale[n][k / 128], the
// engine's q8 format) or per output row (s(n, k) = scale[n]), or fp32 (scale 1). HBM-bound on W: every weight byte is
// read once (group scales add 4 bytes per 128).
//
// Reference: the engine's int8 `matvec` (engine/kernels.js:57-90, q8 weights of engine/kernels.js:15-47) and its MLP
// path with the neuron hook (`swiglu`, engine/kernels_qwen35.js:250-279: a[m, n] = silu(gate) * up, then for each
// push of the layer whose neuron is n or every neuron, add or multiply by the push's value for the row; the row index
// is clamped to 3).
//
// Layout: a tile is 4 R output rows (the launcher takes R = 4: 32-row tiles measured slower in the decode step) and a
// block NW = 4 or 8 waves. Lane (g, j) = (lane / 16, lane % 16) works on rows g, g + 4, ..., g + 4 (R - 1) of the
// tile and on input slot j of every K step: a K step is 16 slots of 16 weight bytes (256 int8 inputs, 64 fp32), so
// one wave load covers 4 rows x 256 contiguous bytes, and the x values of a slot (read from LDS, where x is staged
// once per block) serve the lane's R rows. The waves take the K steps round
// robin, each with all of its weight loads in flight at once. Per-row sums: a 16-lane DPP row reduction, then across
// the waves in LDS. Epilogues: store, accumulate into y (the residual add after down_proj), or SwiGLU over interleaved
// (gate, up) row pairs with the neuron pushes applied (gate_up_proj). With group scales a lane's 16 weights of a K step
// lie in one group (group 2 step + slot / 8), so the lane scales its partial sum of the step once.
// TL: a block takes tiles blockIdx.x, blockIdx.x + gridDim.x, ... (the LM head's 9496 tiles run on a capped grid);
// the next tile's weights are issued before the current tile's products when a wave has one K step per tile (two
// register sets), else before its reduction.
// Split K: an accumulating product without the norm prologue may split its K steps over gridDim.y blocks per 16 rows
// (a product with few output rows, e.g. N = 1024, has too few blocks to draw bandwidth from every CU); each block
// stages and reads only its share of x and W and adds its sums into y with fp32 atomics, so the order of the
// additions, and the last bits of y, may differ between runs.
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

enum GemvEpi : int { kEpiStore = 0, kEpiAccumulate = 1, kEpiSwiglu = 2, kEpiConv = 3 };
constexpr int kEpiAccumulateFixed = 4;  // entry-point code: accumulate, every output summed in one fixed order
constexpr int kGemvConvMaxK = 8;  // conv taps supported by the conv epilogue
constexpr int kGemvHead = 128;    // head size of the gated-norm prologue

// Operands of the gated-norm prologue (GN) and of the conv epilogue (kEpiConv); unused by the other forms.
struct GemvAux {
  const float* z;    // GN: gate rows z[m * ldz + k]
  int64_t ldz;
  const float* hs;   // GN: per-head scale (may be NULL)
  const float* cw;   // conv: weights [cc][ck]
  const float* cb;   // conv: bias [cc] (may be NULL)
  float* cst;        // conv: state [M][ck - 1][cc]
  int cc, ck;        // conv: channels (outputs 0 .. cc - 1 are convolved), taps
  float* cap;        // SwiGLU: activation capture (may be NULL): row m, neuron n at
  int64_t ldc, ldcr; //   cap[(m / T) ldcr + (m % T) ldc + n]
  unsigned long long* amax;  // store: per-row argmax keys (may be NULL), see amax_key
};

// Argmax key of output n with value v: the order-preserving bits of v above the complement of n, so that the largest
// key is the largest value and, among equal values, the lowest index (as argmax_rows_kernel and torch.argmax). -0
// ranks as +0; NaN gets 0, the empty key, and never wins (the scan's strict comparisons). A real key is never 0.
__device__ __forceinline__ unsigned long long amax_key(float v, int n) {
  if (!(v == v)) return 0ull;
  if (v == 0.f) v = 0.f;
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (0xFFFFFFFFu - (uint32_t)n);
}

__device__ __forceinline__ float gsilu(float x) { return silu_f(x); }

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

// sum over the 16 lanes of a DPP row (lanes 16 r .. 16 r + 15), result in every lane of the row
__device__ __forceinline__ float row16_sum_f(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  return v + dpp_f<0x140>(v);  // row_mirror
}

// NORM: x is a residual row; the kernel adds xadd (may be NULL), writes the sum to xout from block 0 (may be NULL),
// and multiplies the RMSNorm of the sum, s * rsqrt(mean s^2 + eps) * (1 + nw), instead of x (HF:720-734).
template <typename TW, int MP, int EPI, int U, bool NORM, bool GS, bool TL, int R = 4, bool GN = false>
__global__ __launch_bounds__(512) void gemv_kernel(const float* __restrict__ x, int64_t ldx, const TW* __restrict__ W,
                                                   const float* __restrict__ wscale, float* __restrict__ y,
                                                   int64_t ldy, int M, int N, int K,
                                                   const q35_push* __restrict__ pushes, int npush, int T,
                                                   const float* __restrict__ xadd, const float* __restrict__ nw,
                                                   float eps, float* __restrict__ xout, GemvAux aux) {
  Q35_ARGS_UPFRONT(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, xadd, nw, eps, xout);
  static_assert(!(GN && NORM), "one prologue");
  static_assert(EPI != kEpiConv || !TL, "the conv epilogue takes one tile per block");
  constexpr int E = WChunk<TW>::kElems;  // weights per lane per 16-byte load
  constexpr int KS = 16 * E;             // inputs per K step
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [MP][K]
  __shared__ float red[TL ? 2 : 1][8][4 * R][MP];  // per-row wave sums (TL: double-buffered over the block's tiles)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NW = blockDim.x >> 6;
  const int g = lane >> 4, j = lane & 15;
  // tiles of 4 R output rows: this block takes tiles blockIdx.x, blockIdx.x + gridDim.x, ...
  const int ntiles = (N + 4 * R - 1) / (4 * R);
  int tile = blockIdx.x;
  // this block's K steps [sb, se) (split K: gridDim.y > 1 only for accumulating products without the norm)
  const int nsplit = gridDim.y;
  const int spb = (K / KS + nsplit - 1) / nsplit;
  const int sb = (int)blockIdx.y * spb, se = min(K / KS, sb + spb);
  if (sb >= se) return;
  const int kb0 = sb * KS, Kb = (se - sb) * KS;  // x columns staged: [kb0, kb0 + Kb)
  static_assert(!GS || E == 16, "group scales are for int8 weights");
  const TW* wr[R];
  const float* sr[R];  // GS: the lane's scale of step 0 in each of its rows (groups of 128 inputs: 2 per K step)
  auto set_rows = [&](int t) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int nr = min(t * 4 * R + g + 4 * r, N - 1);
      wr[r] = W + (size_t)nr * K + j * E;
      sr[r] = GS ? wscale + (size_t)nr * (K >> 7) + (j >> 3) : nullptr;
    }
  };
  set_rows(tile);
  // this wave's K steps: sb + wave, sb + wave + NW, ...; U of them in flight per round. Loads complete in issue order, so the
  // thread's first x chunk (L2) is issued ahead of the first round of weights (HBM): the staging then waits for x
  // only, and its work overlaps the weights' flight
  WChunk<TW> wc[U][R];
  float wsc[U][R];
  auto issue = [&](int s0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = min(s0 + u * NW, se - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        wc[u][r].load(wr[r] + st * KS);
        if (GS) wsc[u][r] = sr[r][2 * st];
      }
    }
  };
  // x (or, with NORM, s = x + xadd times (1 + nw)) into LDS; with NORM each wave also sums the squares of s per row
  // (all loads of a thread go out together: one round trip), the rows' rsqrt factors applied in the epilogue
  __shared__ float ssw[8][MP];
  // the first chunk's operands (k = 4 tid; zero past K), loaded before the weights
  const int kf = 4 * tid;
  f32x4 fv[MP], fa[MP], fw = zero4();
#pragma unroll
  for (int m = 0; m < MP; ++m) {
    fv[m] = zero4();
    fa[m] = zero4();
  }
  if (NORM) {
    if (kf < K) {
      fw = *reinterpret_cast<const f32x4*>(nw + kf);
#pragma unroll
      for (int m = 0; m < MP; ++m) {
        if (m < M) fv[m] = *reinterpret_cast<const f32x4*>(x + m * ldx + kf);
        if (m < M && xadd) fa[m] = *reinterpret_cast<const f32x4*>(xadd + m * ldx + kf);
      }
    }
  } else {
    // the non-NORM staging takes element quads i = tid, tid + blockDim ... of the flattened [MP][Kb]
    const int m0 = kf / Kb, k0 = kf - m0 * Kb;
    if (m0 < M && kf < MP * Kb) fv[0] = *reinterpret_cast<const f32x4*>(x + m0 * ldx + kb0 + k0);
  }
  // GN: the gated norm's operands of the thread's first kGnPre chunks (o, z, the norm weight, the head scale), all
  // loaded before the weights, so that the staging does not wait behind them
  constexpr int kGnPre = GN ? 2 : 1;
  f32x4 go[kGnPre], gz[kGnPre], gw[kGnPre];
  float gh[kGnPre];
  if constexpr (GN) {
#pragma unroll
    for (int j = 0; j < kGnPre; ++j) {
      go[j] = zero4(); gz[j] = zero4(); gw[j] = zero4(); gh[j] = 1.f;
      const int i = tid + j * (int)blockDim.x;
      const int m = (4 * i) / Kb, kk = kb0 + 4 * i - m * Kb;
      if (i < MP * Kb / 4 && m < M) {
        go[j] = *reinterpret_cast<const f32x4*>(x + m * ldx + kk);
        gz[j] = *reinterpret_cast<const f32x4*>(aux.z + m * aux.ldz + kk);
        gw[j] = *reinterpret_cast<const f32x4*>(nw + (kk & (kGemvHead - 1)));
        if (aux.hs) gh[j] = aux.hs[kk / kGemvHead];
      }
    }
  }
  issue(sb + wave);
  // kEpiConv: the epilogue thread of (output row rr, row m) holds its channel's taps, bias and conv state, loaded
  // behind the weights (the epilogue needs the weights' products first anyway)
  float cvw[kGemvConvMaxK], cvs[kGemvConvMaxK - 1], cvb = 0.f;
  if constexpr (EPI == kEpiConv) {
#pragma unroll
    for (int i = 0; i < kGemvConvMaxK; ++i) cvw[i] = 0.f;
#pragma unroll
    for (int i = 0; i < kGemvConvMaxK - 1; ++i) cvs[i] = 0.f;
    const int rr = tid / MP, m = tid - rr * MP, nn = blockIdx.x * 4 * R + rr;
    if (tid < 4 * R * MP && m < M && nn < aux.cc) {
#pragma unroll
      for (int i = 0; i < kGemvConvMaxK; ++i)
        if (i < aux.ck) cvw[i] = aux.cw[(size_t)nn * aux.ck + i];
#pragma unroll
      for (int i = 0; i < kGemvConvMaxK - 1; ++i)
        if (i < aux.ck - 1) cvs[i] = aux.cst[((size_t)m * (aux.ck - 1) + i) * aux.cc + nn];
      if (aux.cb) cvb = aux.cb[nn];
    }
  }
  asm volatile("" ::: "memory");
  if (NORM) {
    float ss[MP];
#pragma unroll
    for (int m = 0; m < MP; ++m) ss[m] = 0.f;
    for (int k = kf; k < K; k += 4 * (int)blockDim.x) {
      const bool first = k == kf;
      const f32x4 w = first ? fw : *reinterpret_cast<const f32x4*>(nw + k);
      f32x4 v[MP];
#pragma unroll
      for (int m = 0; m < MP; ++m) {
        v[m] = zero4();
        if (m < M) v[m] = first ? fv[m] : *reinterpret_cast<const f32x4*>(x + m * ldx + k);
      }
      if (xadd) {
#pragma unroll
        for (int m = 0; m < MP; ++m) {
          if (m < M) {
            const f32x4 a = first ? fa[m] : *reinterpret_cast<const f32x4*>(xadd + m * ldx + k);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[m][e] += a[e];
          }
        }
      }
#pragma unroll
      for (int m = 0; m < MP; ++m) {
        if (xout && blockIdx.x == 0 && m < M) *reinterpret_cast<f32x4*>(xout + m * ldx + k) = v[m];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ss[m] += v[m][e] * v[m][e];
          v[m][e] *= 1.f + w[e];
        }
        *reinterpret_cast<f32x4*>(xs + m * K + k) = v[m];
      }
    }
#pragma unroll
    for (int m = 0; m < MP; ++m) {
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) ss[m] += __shfl_xor(ss[m], off, 64);
      if (lane == 0) ssw[wave][m] = ss[m];
    }
  } else if (GN) {
    // gated RMSNorm per head of 128 inputs (the fused GDN decode step's order): x * r * w * silu(z) * hs, with
    // r = rsqrt(mean x^2 + eps) over the head. Kb and kb0 are multiples of 128, so the 32 quads of a head are 32
    // consecutive i: one half wave, reduced with shuffles inside it (a half wave is wholly in or out of the loop)
    for (int j = 0, i = tid; i < MP * Kb / 4; ++j, i += blockDim.x) {
      const int m = (4 * i) / Kb, k = 4 * i - m * Kb, kk = kb0 + k;
      f32x4 o = zero4(), zz = zero4(), w = zero4();
      float hsc = 1.f;
      if (j < kGnPre) {
#pragma unroll
        for (int jj = 0; jj < kGnPre; ++jj)
          if (jj == j) { o = go[jj]; zz = gz[jj]; w = gw[jj]; hsc = gh[jj]; }
      } else if (m < M) {
        o = *reinterpret_cast<const f32x4*>(x + m * ldx + kk);
        zz = *reinterpret_cast<const f32x4*>(aux.z + m * aux.ldz + kk);
        w = *reinterpret_cast<const f32x4*>(nw + (kk & (kGemvHead - 1)));
        if (aux.hs) hsc = aux.hs[kk / kGemvHead];
      }
      float ss = o[0] * o[0] + o[1] * o[1] + o[2] * o[2] + o[3] * o[3];
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) ss += __shfl_xor(ss, off, 64);
      const float r = rsqrtf(ss * (1.f / kGemvHead) + eps);
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = w[e] * (o[e] * r) * gsilu(zz[e]) * hsc;
      *reinterpret_cast<f32x4*>(xs + m * Kb + k) = v;
    }
  } else {
    for (int i = tid; i < MP * Kb / 4; i += blockDim.x) {
      const int m = (4 * i) / Kb, k = 4 * i - m * Kb;
      f32x4 v = zero4();
      if (m < M) v = i == tid ? fv[0] : *reinterpret_cast<const f32x4*>(x + m * ldx + kb0 + k);
      *reinterpret_cast<f32x4*>(xs + m * Kb + k) = v;
    }
  }
  __syncthreads();
  // NORM: row m's rsqrt(mean s^2 + eps) factor (TL: once per block, else in the epilogue)
  auto rs = [&](int m) {
    float ss = 0.f;
    for (int w = 0; w < NW; ++w) ss += ssw[w][m];
    return rsqrtf(ss / (float)K + eps);
  };
  float rsf[MP];
  if (NORM && TL) {
#pragma unroll
    for (int m = 0; m < MP; ++m) rsf[m] = rs(m);
  }
  // acc += this wave's K step st over the lane's rows, weights (and group scales) from w (ws)
  auto mac = [&](const WChunk<TW>(&w)[R], const float(&ws)[R], int st, float(&acc)[R][MP]) {
    const int k = (st - sb) * KS + j * E;  // column in the staged x (Kb == K without a split)
    float part[R][MP];                     // GS: this step's sums, scaled once by the group's scale
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MP; ++m) part[r][m] = 0.f;
#pragma unroll
    for (int c = 0; c < E; c += 4) {
      f32x4 xv[MP];
#pragma unroll
      for (int m = 0; m < MP; ++m) xv[m] = *reinterpret_cast<const f32x4*>(xs + m * Kb + k + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float wv = w[r].at(c + e);
#pragma unroll
          for (int m = 0; m < MP; ++m) {
            if (GS) part[r][m] += wv * xv[m][e];
            else acc[r][m] += wv * xv[m][e];
          }
        }
      }
    }
    if (GS) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MP; ++m) acc[r][m] += ws[r] * part[r][m];
    }
  };
  // store with aux.amax: the best argmax key of this thread's (output row, x row) over the block's tiles
  unsigned long long best_key = 0ull;
  // the tile's row sums across the waves and its epilogue. red[it & 1] is rewritten two tiles later, after a barrier
  // that every thread reaches only past this tile's epilogue
  auto finish = [&](int it, int n0, float(&acc)[R][MP]) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MP; ++m) acc[r][m] = row16_sum_f(acc[r][m]);
    float(*rd)[4 * R][MP] = red[TL ? it & 1 : 0];
    if (j == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MP; ++m) rd[wave][g + 4 * r][m] = acc[r][m];
    }
    __syncthreads();
    auto rowsum = [&](int rr, int m) {
      float p[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) p[w] = w < NW ? rd[w][rr][m] : 0.f;
      float v = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      return NORM ? v * (TL ? rsf[m] : rs(m)) : v;
    };
    if (EPI != kEpiSwiglu) {
      if (tid < 4 * R * MP) {
        const int rr = tid / MP, m = tid - rr * MP;
        const int nn = n0 + rr;
        if (m < M && nn < N) {
          float v = rowsum(rr, m);
          if (wscale && !GS) v *= wscale[nn];
          float* dst = y + m * ldy + nn;
          if (EPI == kEpiConv && nn < aux.cc) {
            // causal conv over the channel's last ck inputs (the conv state, then v) + SiLU; state <- [rows 1.. | v]
            float a = cvb;
#pragma unroll
            for (int i = 0; i < kGemvConvMaxK; ++i) {
              if (i >= aux.ck) break;
              a += cvw[i] * (i < aux.ck - 1 ? cvs[i] : v);
            }
            float* cs = aux.cst + (size_t)m * (aux.ck - 1) * aux.cc + nn;
#pragma unroll
            for (int i = 0; i < kGemvConvMaxK - 1; ++i) {
              if (i >= aux.ck - 1) break;
              cs[(size_t)i * aux.cc] = i + 1 < aux.ck - 1 ? cvs[i + 1] : v;
            }
            *dst = silu_f(a);
          } else if (EPI == kEpiAccumulate && nsplit > 1) {
            __hip_atomic_fetch_add(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          } else {
            *dst = EPI == kEpiAccumulate ? *dst + v : v;
            if (EPI == kEpiStore && aux.amax) {
              const unsigned long long kk = amax_key(v, nn);
              best_key = kk > best_key ? kk : best_key;
            }
          }
        }
      }
    } else {
      // rows 2 q and 2 q + 1 of the tile are gate and up of neuron n0 / 2 + q
      if (tid < 2 * R * MP) {
        const int qn = tid / MP, m = tid - qn * MP;
        const int ng = n0 + 2 * qn;
        const int neuron = ng >> 1;
        if (m < M && ng + 1 < N) {
          float gt = rowsum(2 * qn, m), up = rowsum(2 * qn + 1, m);
          if (wscale && !GS) { gt *= wscale[ng]; up *= wscale[ng + 1]; }
          float a = gsilu(gt) * up;
          const int row = min(m / T, 3);
          for (int p = 0; p < npush; ++p) a = apply_push(pushes + p, neuron, row, a);
          y[m * ldy + neuron] = a;
          if (aux.cap) aux.cap[(int64_t)(m / T) * aux.ldcr + (int64_t)(m % T) * aux.ldc + neuron] = a;
        }
      }
    }
  };
  if constexpr (!TL) {
    // one tile per block
    float acc[R][MP];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MP; ++m) acc[r][m] = 0.f;
    for (int s0 = sb + wave; s0 < se; s0 += U * NW) {
      if (s0 != sb + wave) issue(s0);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int st = s0 + u * NW;
        if (st >= se) break;
        mac(wc[u], wsc[u], st, acc);
      }
    }
    finish(0, tile * 4 * R, acc);
  } else if constexpr (U == 1) {
    // at most one K step per wave and tile: the next tile's weights go out before this tile's products, into the
    // other of two register sets, so two tiles' loads are in flight while the wave computes
    const int st = sb + wave;
    const bool has = st < se;
    WChunk<TW> wb[R];
    float wbs[R];
    auto one = [&](int it, const WChunk<TW>(&cur)[R], const float(&cs)[R], WChunk<TW>(&nx)[R], float(&ns)[R]) {
      const int next = tile + (int)gridDim.x;
      if (next < ntiles) {
        set_rows(next);
        const int sl = min(st, se - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          nx[r].load(wr[r] + sl * KS);
          if (GS) ns[r] = sr[r][2 * sl];
        }
      }
      float acc[R][MP];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MP; ++m) acc[r][m] = 0.f;
      if (has) mac(cur, cs, st, acc);
      finish(it, tile * 4 * R, acc);
      tile = next;
      return next < ntiles;
    };
    for (int it = 0;; it += 2) {
      if (!one(it, wc[0], wsc[0], wb, wbs)) break;
      if (!one(it + 1, wb, wbs, wc[0], wsc[0])) break;
    }
  } else {
    for (int it = 0;; ++it) {
      float acc[R][MP];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MP; ++m) acc[r][m] = 0.f;
      for (int s0 = sb + wave; s0 < se; s0 += U * NW) {
        if (s0 != sb + wave) issue(s0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int st = s0 + u * NW;
          if (st >= se) break;
          mac(wc[u], wsc[u], st, acc);
        }
      }
      // the next tile's first round of weights goes out before this tile's reduction and epilogue
      const int next = tile + (int)gridDim.x;
      if (next < ntiles) {
        set_rows(next);
        issue(sb + wave);
      }
      finish(it, tile * 4 * R, acc);
      if (next >= ntiles) break;
      tile = next;
    }
  }
  if constexpr (EPI == kEpiStore) {
    if (aux.amax) {  // uniform: every thread reaches the barrier
      // the block's best key per row of x, then one device-scope atomic max per row
      __shared__ unsigned long long kbest[4 * R * MP];
      if (tid < 4 * R * MP) kbest[tid] = best_key;
      __syncthreads();
      if (tid < MP && tid < M) {
        unsigned long long k = 0ull;
        for (int rr = 0; rr < 4 * R; ++rr) k = kbest[rr * MP + tid] > k ? kbest[rr * MP + tid] : k;
        if (k) __hip_atomic_fetch_max(aux.amax + tid, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// The argmax keys of q35_gemv_norm_argmax turned into indices (the empty key: index 0, as argmax_rows_kernel reports
// for a row that nothing wins), and the slots cleared for the next call.
__global__ __launch_bounds__(64) void amax_take_kernel(unsigned long long* __restrict__ slots, int rows,
                                                       int32_t* __restrict__ idx) {
  const int r = threadIdx.x;
  if (r < rows) {
    const unsigned long long k = slots[r];
    idx[r] = k ? (int32_t)(0xFFFFFFFFu - (uint32_t)k) : 0;
    slots[r] = 0ull;
  }
}

// a[m, n] = silu(gu[m, n]) * gu[m, I + n] with the pushes applied (the prefill form over a [gate | up] projection)
__global__ __launch_bounds__(256) void swiglu_push_kernel(const float* __restrict__ gu, float* __restrict__ a,
                                                          int64_t M, int I, const q35_push* __restrict__ pushes,
                                                          int npush, int T, float* __restrict__ cap, int64_t ldc,
                                                          int64_t ldcr) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * I) return;
  const int64_t m = i / I;
  const int n = (int)(i - m * I);
  float v = gsilu(gu[m * 2 * I + n]) * gu[m * 2 * I + I + n];
  const int row = (int)min(m / T, (int64_t)3);
  for (int p = 0; p < npush; ++p) v = apply_push(pushes + p, n, row, v);
  a[i] = v;
  if (cap) cap[(m / T) * ldcr + (m % T) * ldc + n] = v;
}

}  // namespace q35

namespace {
// Blocks of 16 output rows at which a product is split over K: below this many, an accumulating product without the
// norm splits its K steps so that blocks x splits reaches it (one block per CU of the MI355X).
constexpr int64_t kGemvSplitTarget = 256;
// Grid cap: a product with more 16-row tiles (the LM head: 9496) loops each block over tiles blockIdx.x,
// + gridDim.x, ... (x staged once per block; four 4-wave blocks per CU at 128 VGPRs). The products with fewer tiles
// take one tile per block, in a kernel without the loop (measured faster for them).
constexpr int64_t kGemvMaxBlocks = 1024;

struct NormArgs {
  const float* xadd;
  const float* nw;
  float eps;
  float* xout;
  q35::GemvAux aux;
};

template <typename TW, int EPI, int U, bool NORM, bool GS, bool GN, int R = 4>
void gemv_launch_u(const float* x, int64_t ldx, const TW* W, const float* wscale, float* y, int64_t ldy, int64_t M,
                   int64_t N, int64_t K, const q35_push* pushes, int npush, int64_t T, int nw, int nsplit,
                   const NormArgs& na, hipStream_t st) {
  using namespace q35;
  const int mp = M <= 1 ? 1 : M <= 2 ? 2 : M <= 3 ? 3 : M <= 4 ? 4 : 8;
  constexpr int KS = 16 * WChunk<TW>::kElems;
  const int64_t spb = (K / KS + nsplit - 1) / nsplit;
  const size_t lds = (size_t)mp * spb * KS * sizeof(float);
  // 8 rows of x: tiles of 8 output rows (R 2), so that the accumulators and weight registers fit without spilling
  constexpr int R8 = R > 2 ? 2 : R;
  const int re = mp == 8 ? R8 : R;
  const int64_t ntiles = (N + 4 * re - 1) / (4 * re);
  const dim3 grid((unsigned)(ntiles < kGemvMaxBlocks ? ntiles : kGemvMaxBlocks), (unsigned)nsplit), block(64 * nw);
#define Q35_GEMV(MP, TL)                                                                                           \
  hipLaunchKernelGGL((gemv_kernel<TW, MP, EPI, U, NORM, GS, TL, (MP == 8 ? R8 : R), GN>), grid, block, lds, st, x, \
                     ldx, W, wscale, y, ldy, (int)M, (int)N, (int)K, pushes, npush, (int)T, na.xadd, na.nw, na.eps,   \
                     na.xout, na.aux)
  if constexpr (EPI == kEpiConv) {  // one tile per block (the entry point bounds N)
    switch (mp) {
      case 1: Q35_GEMV(1, false); break;
      case 2: Q35_GEMV(2, false); break;
      case 3: Q35_GEMV(3, false); break;
      case 4: Q35_GEMV(4, false); break;
      default: if constexpr (U <= 2) Q35_GEMV(8, false); break;  // 8 rows: U <= 2 (gemv_launch)
    }
  } else if (ntiles > kGemvMaxBlocks) {
    switch (mp) {
      case 1: Q35_GEMV(1, true); break;
      case 2: Q35_GEMV(2, true); break;
      case 3: Q35_GEMV(3, true); break;
      case 4: Q35_GEMV(4, true); break;
      default: if constexpr (U <= 2) Q35_GEMV(8, true); break;  // 8 rows: U <= 2 (gemv_launch)
    }
  } else {
    switch (mp) {
      case 1: Q35_GEMV(1, false); break;
      case 2: Q35_GEMV(2, false); break;
      case 3: Q35_GEMV(3, false); break;
      case 4: Q35_GEMV(4, false); break;
      default: if constexpr (U <= 2) Q35_GEMV(8, false); break;  // 8 rows: U <= 2 (gemv_launch)
    }
  }
#undef Q35_GEMV
}


// 4 waves when a block has at most 4 K steps, else 8; each wave's steps all in flight at once up to 4
// fixed (epilogue 4, accumulate in a fixed order): no split over K; a product with too few 16-row tiles to occupy the
// device takes 4-row tiles instead (the stack's N = 1024 products: 256 blocks), each block over all of K, so every
// output is summed in one order whatever the run (0.6-1.4 us slower per call than the split at N = 1024, M = 3)
template <typename TW, int EPI, bool NORM, bool GS = false, bool GN = false>
int gemv_launch(const float* x, int64_t ldx, const TW* W, const float* wscale, float* y, int64_t ldy, int64_t M,
                int64_t N, int64_t K, const q35_push* pushes, int npush, int64_t T, const NormArgs& na,
                hipStream_t st, bool fixed = false) {
  using namespace q35;
  const int64_t steps = K / (16 * WChunk<TW>::kElems);
  const int64_t nblk = (N + 15) / 16;
  int64_t nsplit = 1;
  if constexpr (EPI == kEpiAccumulate && !NORM) if (fixed && nblk < kGemvSplitTarget && (N + 3) / 4 <= kGemvMaxBlocks) {
    const int nw = steps <= 4 ? 4 : 8;
    const int64_t per_wave = (steps + nw - 1) / nw;
    if (per_wave <= 1)
      gemv_launch_u<TW, EPI, 1, NORM, GS, GN, 1>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, nw, 1, na, st);
    else if (per_wave <= 2 || M > 4)
      gemv_launch_u<TW, EPI, 2, NORM, GS, GN, 1>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, nw, 1, na, st);
    else
      gemv_launch_u<TW, EPI, 4, NORM, GS, GN, 1>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, nw, 1, na, st);
    return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
  }
  if (EPI == kEpiAccumulate && !NORM && !fixed && nblk < kGemvSplitTarget) {
    nsplit = (kGemvSplitTarget + nblk - 1) / nblk;
    if (nsplit > steps) nsplit = steps;
    if (nsplit > 65535) nsplit = 65535;
    const int64_t spb = (steps + nsplit - 1) / nsplit;
    nsplit = (steps + spb - 1) / spb;  // no empty split
  }
  const int64_t bsteps = (steps + nsplit - 1) / nsplit;
  const int nw = bsteps <= 4 ? 4 : 8;
  const int64_t per_wave = (bsteps + nw - 1) / nw;
  // more than 4 rows of x: at most two K steps per wave in flight (four spill the registers of 8 rows)
  if (per_wave <= 1)
    gemv_launch_u<TW, EPI, 1, NORM, GS, GN>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, nw, (int)nsplit, na, st);
  else if (per_wave <= 2)
    gemv_launch_u<TW, EPI, 2, NORM, GS, GN>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, nw, (int)nsplit, na, st);
  else if (M > 4)
    gemv_launch_u<TW, EPI, 2, NORM, GS, GN>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, nw, (int)nsplit, na, st);
  else
    gemv_launch_u<TW, EPI, 4, NORM, GS, GN>(x, ldx, W, wscale, y, ldy, M, N, K, pushes, npush, T, nw, (int)nsplit, na, st);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

template <bool NORM>
int gemv_dispatch(const float* x, int64_t ldx, const void* W, int w_dtype, const float* w_scale, float* y,
                  int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes, int np,
                  int64_t T, const NormArgs& na, hipStream_t st) {
  using namespace q35;
  const bool fx = epilogue == kEpiAccumulateFixed;
  const bool acc = epilogue == kEpiAccumulate || fx;
  if (w_dtype == Q35_I8_G128) {
    const int8_t* w8 = (const int8_t*)W;
    if (epilogue == kEpiStore) return gemv_launch<int8_t, kEpiStore, NORM, true>(x, ldx, w8, w_scale, y, ldy, M, N, K, pushes, np, T, na, st);
    if (acc) return gemv_launch<int8_t, kEpiAccumulate, NORM, true>(x, ldx, w8, w_scale, y, ldy, M, N, K, pushes, np, T, na, st, fx);
    return gemv_launch<int8_t, kEpiSwiglu, NORM, true>(x, ldx, w8, w_scale, y, ldy, M, N, K, pushes, np, T, na, st);
  }
  if (w_dtype == Q35_I8) {
    const int8_t* w8 = (const int8_t*)W;
    if (epilogue == kEpiStore) return gemv_launch<int8_t, kEpiStore, NORM>(x, ldx, w8, w_scale, y, ldy, M, N, K, pushes, np, T, na, st);
    if (acc) return gemv_launch<int8_t, kEpiAccumulate, NORM>(x, ldx, w8, w_scale, y, ldy, M, N, K, pushes, np, T, na, st, fx);
    return gemv_launch<int8_t, kEpiSwiglu, NORM>(x, ldx, w8, w_scale, y, ldy, M, N, K, pushes, np, T, na, st);
  }
  const float* wf = (const float*)W;
  if (epilogue == kEpiStore) return gemv_launch<float, kEpiStore, NORM>(x, ldx, wf, w_scale, y, ldy, M, N, K, pushes, np, T, na, st);
  if (acc) return gemv_launch<float, kEpiAccumulate, NORM>(x, ldx, wf, w_scale, y, ldy, M, N, K, pushes, np, T, na, st, fx);
  return gemv_launch<float, kEpiSwiglu, NORM>(x, ldx, wf, w_scale, y, ldy, M, N, K, pushes, np, T, na, st);
}

// argument checks shared by the two entry points
int gemv_check(const float* x, int64_t ldx, const void* W, int w_dtype, const float* w_scale, float* y, int64_t ldy,
               int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes, int64_t npush, int64_t T,
               const float* cap = nullptr, int64_t ldc = 0, int64_t ldcr = 0) {
  using namespace q35;
  if (!x || !W || !y || M <= 0 || N <= 0 || K <= 0 || ldx < K || T <= 0) return Q35_EINVAL;
  if (cap && (epilogue != kEpiSwiglu || ldc < N / 2 || ldcr < N / 2 || ((uintptr_t)cap & 3))) return Q35_EINVAL;
  if (w_dtype == Q35_I8_G128 && !w_scale) return Q35_EINVAL;
  if (npush < 0 || (npush > 0 && !pushes)) return Q35_EINVAL;
  if (epilogue == kEpiSwiglu ? (N & 1) || ldy < N / 2 : ldy < N) return Q35_EINVAL;
  if (epilogue != kEpiStore && epilogue != kEpiAccumulate && epilogue != kEpiSwiglu &&
      epilogue != kEpiAccumulateFixed)
    return Q35_EINVAL;
  if (w_dtype != Q35_I8 && w_dtype != Q35_I8_G128 && w_dtype != Q35_F32) return Q35_EUNSUPPORTED;
  if (M > 8 || (K % 256) != 0 || (ldx & 3) || ((uintptr_t)x & 15) || ((uintptr_t)W & 15)) return Q35_EUNSUPPORTED;
  const int mp = M <= 1 ? 1 : M <= 2 ? 2 : M <= 3 ? 3 : M <= 4 ? 4 : 8;
  if ((int64_t)mp * K * 4 > 64 * 1024 || N > 0x7fffffff || npush > 64) return Q35_EUNSUPPORTED;
  return Q35_OK;
}
}  // namespace

extern "C" int q35_gemv(const float* x, int64_t ldx, const void* W, int w_dtype, const float* w_scale, float* y,
                        int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes,
                        int64_t npush, int64_t T, float* cap, int64_t ld_cap, int64_t ld_cap_row,
                        q35_stream_t stream) {
  const int chk = gemv_check(x, ldx, W, w_dtype, w_scale, y, ldy, M, N, K, epilogue, pushes, npush, T, cap, ld_cap,
                             ld_cap_row);
  if (chk != Q35_OK) return chk;
  NormArgs na = {nullptr, nullptr, 0.f, nullptr, {}};
  na.aux.cap = cap;
  na.aux.ldc = ld_cap;
  na.aux.ldcr = ld_cap_row;
  return gemv_dispatch<false>(x, ldx, W, w_dtype, w_scale, y, ldy, M, N, K, epilogue, pushes, (int)npush, T, na,
                              reinterpret_cast<hipStream_t>(stream));
}

extern "C" int q35_gemv_norm(const float* x, const float* x_add, float* x_out, int64_t ldx, const float* norm_w,
                             float eps, const void* W, int w_dtype, const float* w_scale, float* y, int64_t ldy,
                             int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes, int64_t npush,
                             int64_t T, float* cap, int64_t ld_cap, int64_t ld_cap_row, q35_stream_t stream) {
  const int chk = gemv_check(x, ldx, W, w_dtype, w_scale, y, ldy, M, N, K, epilogue, pushes, npush, T, cap, ld_cap,
                             ld_cap_row);
  if (chk != Q35_OK) return chk;
  if (!norm_w) return Q35_EINVAL;
  if (((uintptr_t)norm_w & 15) || (x_add && ((uintptr_t)x_add & 15)) || (x_out && ((uintptr_t)x_out & 15)))
    return Q35_EUNSUPPORTED;
  // x_out is written while other blocks still read x and x_add: it must not overlap them
  auto overlap = [&](const float* a) {
    return a && x_out && a < x_out + (M - 1) * ldx + K && x_out < a + (M - 1) * ldx + K;
  };
  if (overlap(x) || overlap(x_add)) return Q35_EINVAL;
  NormArgs na = {x_add, norm_w, eps, x_out, {}};
  na.aux.cap = cap;
  na.aux.ldc = ld_cap;
  na.aux.ldcr = ld_cap_row;
  return gemv_dispatch<true>(x, ldx, W, w_dtype, w_scale, y, ldy, M, N, K, epilogue, pushes, (int)npush, T, na,
                             reinterpret_cast<hipStream_t>(stream));
}

extern "C" int q35_gemv_norm_argmax(const float* x, const float* x_add, float* x_out, int64_t ldx,
                                    const float* norm_w, float eps, const void* W, int w_dtype, const float* w_scale,
                                    float* y, int64_t ldy, int64_t M, int64_t N, int64_t K, uint64_t* slots,
                                    int32_t* idx, q35_stream_t stream) {
  using namespace q35;
  const int chk = gemv_check(x, ldx, W, w_dtype, w_scale, y, ldy, M, N, K, kEpiStore, nullptr, 0, 1);
  if (chk != Q35_OK) return chk;
  if (!norm_w || !slots || !idx) return Q35_EINVAL;
  if (((uintptr_t)norm_w & 15) || (x_add && ((uintptr_t)x_add & 15)) || (x_out && ((uintptr_t)x_out & 15)) ||
      ((uintptr_t)slots & 7) || ((uintptr_t)idx & 3))
    return Q35_EUNSUPPORTED;
  auto overlap = [&](const float* a) {
    return a && x_out && a < x_out + (M - 1) * ldx + K && x_out < a + (M - 1) * ldx + K;
  };
  if (overlap(x) || overlap(x_add)) return Q35_EINVAL;
  NormArgs na = {x_add, norm_w, eps, x_out, {}};
  na.aux.amax = reinterpret_cast<unsigned long long*>(slots);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int r = gemv_dispatch<true>(x, ldx, W, w_dtype, w_scale, y, ldy, M, N, K, kEpiStore, nullptr, 0, 1, na, st);
  if (r != Q35_OK) return r;
  hipLaunchKernelGGL(amax_take_kernel, dim3(1), dim3(64), 0, st, reinterpret_cast<unsigned long long*>(slots),
                     (int)M, idx);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

extern "C" int q35_gemv_norm_conv(const float* x, const float* x_add, float* x_out, int64_t ldx,
                                  const float* norm_w, float eps, const void* W, int w_dtype, const float* w_scale,
                                  float* y, int64_t ldy, int64_t M, int64_t N, int64_t K, const float* conv_w,
                                  const float* conv_bias, float* conv_state, int64_t conv_channels, int64_t conv_k,
                                  q35_stream_t stream) {
  using namespace q35;
  const int chk = gemv_check(x, ldx, W, w_dtype, w_scale, y, ldy, M, N, K, kEpiStore, nullptr, 0, 1);
  if (chk != Q35_OK) return chk;
  if (!norm_w || !conv_w || !conv_state || conv_channels <= 0 || conv_channels > N || conv_k < 2) return Q35_EINVAL;
  // one tile per block: 16 output rows, or 8 for more than 4 rows of x
  if (conv_k > kGemvConvMaxK || (N + (M > 4 ? 7 : 15)) / (M > 4 ? 8 : 16) > kGemvMaxBlocks ||
      conv_channels * conv_k > 0x7fffffff)
    return Q35_EUNSUPPORTED;
  if (((uintptr_t)norm_w & 15) || (x_add && ((uintptr_t)x_add & 15)) || (x_out && ((uintptr_t)x_out & 15)))
    return Q35_EUNSUPPORTED;
  auto overlap = [&](const float* a) {
    return a && x_out && a < x_out + (M - 1) * ldx + K && x_out < a + (M - 1) * ldx + K;
  };
  if (overlap(x) || overlap(x_add)) return Q35_EINVAL;
  NormArgs na = {x_add, norm_w, eps, x_out, {}};
  na.aux.cw = conv_w;
  na.aux.cb = conv_bias;
  na.aux.cst = conv_state;
  na.aux.cc = (int)conv_channels;
  na.aux.ck = (int)conv_k;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (w_dtype == Q35_I8_G128)
    return gemv_launch<int8_t, kEpiConv, true, true>(x, ldx, (const int8_t*)W, w_scale, y, ldy, M, N, K, nullptr, 0,
                                                      1, na, st);
  if (w_dtype == Q35_I8)
    return gemv_launch<int8_t, kEpiConv, true>(x, ldx, (const int8_t*)W, w_scale, y, ldy, M, N, K, nullptr, 0, 1, na,
                                               st);
  return gemv_launch<float, kEpiConv, true>(x, ldx, (const float*)W, w_scale, y, ldy, M, N, K, nullptr, 0, 1, na, st);
}

extern "C" int q35_gemv_gated_norm(const float* o, int64_t ldo, const float* z, int64_t ldz, const float* norm_w,
                                   const float* head_scale, float eps, const void* W, int w_dtype,
                                   const float* w_scale, float* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                                   int epilogue, q35_stream_t stream) {
  using namespace q35;
  const int chk = gemv_check(o, ldo, W, w_dtype, w_scale, y, ldy, M, N, K, epilogue, nullptr, 0, 1);
  if (chk != Q35_OK) return chk;
  if (!z || !norm_w || ldz < K ||
      (epilogue != kEpiStore && epilogue != kEpiAccumulate && epilogue != kEpiAccumulateFixed))
    return Q35_EINVAL;
  const bool fx = epilogue == kEpiAccumulateFixed;
  // the prologue normalises whole heads of 128 inputs: int8 weights (K steps of 256) keep every split head-aligned
  if (w_dtype == Q35_F32) return Q35_EUNSUPPORTED;
  if ((ldz & 3) || ((uintptr_t)z & 15) || ((uintptr_t)norm_w & 15)) return Q35_EUNSUPPORTED;
  NormArgs na = {nullptr, norm_w, eps, nullptr, {}};
  na.aux.z = z;
  na.aux.ldz = ldz;
  na.aux.hs = head_scale;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int8_t* w8 = (const int8_t*)W;
  if (w_dtype == Q35_I8_G128) {
    if (epilogue == kEpiStore)
      return gemv_launch<int8_t, kEpiStore, false, true, true>(o, ldo, w8, w_scale, y, ldy, M, N, K, nullptr, 0, 1,
                                                               na, st);
    return gemv_launch<int8_t, kEpiAccumulate, false, true, true>(o, ldo, w8, w_scale, y, ldy, M, N, K, nullptr, 0, 1,
                                                                  na, st, fx);
  }
  if (epilogue == kEpiStore)
    return gemv_launch<int8_t, kEpiStore, false, false, true>(o, ldo, w8, w_scale, y, ldy, M, N, K, nullptr, 0, 1, na,
                                                              st);
  return gemv_launch<int8_t, kEpiAccumulate, false, false, true>(o, ldo, w8, w_scale, y, ldy, M, N, K, nullptr, 0, 1,
                                                                 na, st, fx);
}

extern "C" int q35_swiglu_push(const float* gu, float* a, int64_t M, int64_t I, const q35_push* pushes,
                               int64_t npush, int64_t T, float* cap, int64_t ld_cap, int64_t ld_cap_row,
                               q35_stream_t stream) {
  using namespace q35;
  if (!gu || !a || M <= 0 || I <= 0 || T <= 0 || npush < 0 || (npush > 0 && !pushes)) return Q35_EINVAL;
  if (cap && (ld_cap < I || ld_cap_row < I || ((uintptr_t)cap & 3))) return Q35_EINVAL;
  if (M * I > ((int64_t)1 << 40) || (M * I + 255) / 256 > 0x7fffffff || npush > 64 || I > 0x7fffffff)
    return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(swiglu_push_kernel, dim3((unsigned)((M * I + 255) / 256)), dim3(256), 0, st, gu, a, M, (int)I,
                     pushes, (int)npush, (int)T, cap, ld_cap, ld_cap_row);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
