// Gated DeltaNet, chunked form (prefill): chunk 64, UT/WY intra-chunk transform, fp32 state carried across chunks.
//
// Math (HF:249-327 torch_chunk_gated_delta_rule; the decay masks and the 63-row forward substitution at HF:288-298).
// Per (b, h) and chunk c of 64 positions, with gamma = cumsum(g) inside the chunk, q^ = l2norm(q) * scale,
// k^ = l2norm(k), and L[t][s] = -beta_t (k^_t . k^_s) exp(gamma_t - gamma_s) for s < t (0 otherwise):
//   T      = (I - L)^-1                                  (HF's substitution loop + eye)
//   U      = T diag(beta) V                              (HF `value`)
//   W      = T diag(beta exp(gamma)) K^                  (HF `k_cumdecay`)
//   P[t][s]= (q^_t . k^_s) exp(gamma_t - gamma_s), s <= t  (HF intra-chunk `attn`)
//   per chunk, in order:  Vn = U - W S ;  O = (Q^ exp(gamma)) S + P Vn ;  S <- exp(gamma_last) S + K~^T Vn
//   with K~[s] = k^_s exp(gamma_last - gamma_s). Every exponent is <= 0 (g <= 0), so nothing overflows.
// The l2 normalisation is applied as fp32 row / column scales of the products (q, k stay exact bf16 MFMA operands).
//
// Kernel 1, gdn_chunk_prep_kernel: one block (4 waves, 64 KB LDS, two blocks per CU) per (chunk, head, row), all
// chunks in parallel. 16-byte loads; K and V are transposed 8x8 in registers into XOR-swizzled LDS tiles (bank-
// conflict-free writes and MFMA-operand reads); K K^T and Q K^T on bf16 MFMA with operands read straight from L2;
// the 64x64 unit-lower-triangular inverse in fp32 (16x16 diagonal blocks by forward substitution in registers, then
// one independent chain per block column for the off-diagonal blocks on fp32 MFMA); U and W on bf16 MFMA. Every
// operand of kernel 2 is written pre-swizzled into MFMA lane order (16 contiguous bytes per lane).
// Kernel 2, gdn_chunk_scan_kernel: one block of 2 waves per (16-column slice of the value dim, head, row).
// Wave 0 carries the 128x16 fp32 state slice in MFMA accumulators through the chunks and does only the serial work
// (Vn = U - W S, S <- e^g S + K~^T Vn), with the next chunk's records copied global -> LDS by global_load_lds one
// chunk ahead (no registers held, explicit vmcnt waits). It hands the packed
// state and Vn of each chunk to wave 1 through a double-buffered LDS slot (one barrier per chunk); wave 1 forms the
// outputs O = Q~ S + P Vn off the serial path. The 8 slices of a head are placed on one XCD to share its L2.
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kC = 64;          // chunk
constexpr int kD = 128;         // Dk = Dv
constexpr int kFS = kC + 4;     // row stride of the [64][64] fp32 LDS array
constexpr int kPS = kC + 8;     // row stride of the [64][64] bf16 P array
constexpr int kWS = kD + 8;     // row stride of the [64][128] bf16 W staging array (aliases the fp32 array)

// Per-(b, h, chunk) workspace records.
constexpr size_t kWElems = 4 * 4 * 64 * 8;   // W   [mt 4][ks 4][lane][8] bf16
constexpr size_t kQElems = 4 * 4 * 64 * 8;   // Q~  [mt 4][ks 4][lane][8] bf16: q rq_t scale exp(gamma_t)
constexpr size_t kKTElems = 8 * 2 * 64 * 8;  // K~^T[mt 8][ks 2][lane][8] bf16
constexpr size_t kPElems = 4 * 2 * 64 * 8;   // P   [mt 4][ks 2][lane][8] bf16
constexpr size_t kUElems = 8 * 4 * 64 * 4;   // U   [slice 8][mt 4][lane][4] fp32
constexpr size_t kEGElems = 64 * 4;          // exp(gamma_last) replicated [lane][4] fp32 (one 1 KB record)

struct ChunkWs {
  __bf16* W;
  __bf16* Q;
  __bf16* KT;
  __bf16* P;
  float* U;
  float* EG;
};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static ChunkWs chunk_ws_layout(void* base, size_t nbhc, size_t* total) {
  ChunkWs w;
  char* p = (char*)base;
  size_t off = 0;
  w.W = (__bf16*)(p + off);  off = align256(off + nbhc * kWElems * 2);
  w.Q = (__bf16*)(p + off);  off = align256(off + nbhc * kQElems * 2);
  w.KT = (__bf16*)(p + off); off = align256(off + nbhc * kKTElems * 2);
  w.P = (__bf16*)(p + off);  off = align256(off + nbhc * kPElems * 2);
  w.U = (float*)(p + off);   off = align256(off + nbhc * kUElems * 4);
  w.EG = (float*)(p + off);  off = align256(off + nbhc * kEGElems * 4);
  *total = off;
  return w;
}

// k index of position p (0..7) of lane group g in a 32-wide K step fed from two 16-row accumulator tiles
__device__ __forceinline__ int kmap(int g, int p) { return p < 4 ? 4 * g + p : 12 + 4 * g + p; }

// Transposed [128][64] bf16 tiles: 16-byte block b (8 positions) of row d lives at block b ^ swz(d).
__device__ __forceinline__ int swz(int d) { return (d ^ (d >> 3)) & 7; }
__device__ __forceinline__ int tofs(int d, int pos) { return d * kC + 8 * ((pos >> 3) ^ swz(d)) + (pos & 7); }

__device__ __forceinline__ bf16x8 load8b(const __bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ bf16x8 load8b(const float* p) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) { r[e] = (__bf16)a[e]; r[4 + e] = (__bf16)b[e]; }
  return r;
}
__device__ __forceinline__ f32x4 load4f(const __bf16* p) {
  const uint2 r = *reinterpret_cast<const uint2*>(p);
  f32x4 o = {bf16lo(r.x), bf16hi(r.x), bf16lo(r.y), bf16hi(r.y)};
  return o;
}
__device__ __forceinline__ f32x4 load4f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// Raw loads as packed bf16 bits (fp32 input rounded to bf16), issued unconditionally from clamped addresses so that
// many loads stay in flight; rows outside the sequence are zeroed afterwards with a select, not a branch (a load
// inside a branch whose result is used in the branch makes the compiler wait for it right there).
__device__ __forceinline__ uint4 raw8(const __bf16* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint4 raw8(const float* p) {
  const bf16x8 r = load8b(p);
  return *reinterpret_cast<const uint4*>(&r);
}
__device__ __forceinline__ uint2 raw4(const __bf16* p) { return *reinterpret_cast<const uint2*>(p); }
__device__ __forceinline__ uint2 raw4(const float* p) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  bf16x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = (__bf16)a[e];
  return *reinterpret_cast<const uint2*>(&r);
}
__device__ __forceinline__ uint4 mask8(uint4 r, bool keep) {
  const uint4 z = {0u, 0u, 0u, 0u};
  return keep ? r : z;
}
__device__ __forceinline__ float sumsq8(const uint4& r) {
  const float x[8] = {bf16lo(r.x), bf16hi(r.x), bf16lo(r.y), bf16hi(r.y),
                      bf16lo(r.z), bf16hi(r.z), bf16lo(r.w), bf16hi(r.w)};
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  return ss;
}
// sum of squares in the input precision (fp32 input: of the unrounded values)
__device__ __forceinline__ float sumsq8_in(const __bf16* p, const uint4& r) { return sumsq8(r); }
__device__ __forceinline__ float sumsq8_in(const float* p, const uint4&) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) ss += a[e] * a[e] + b[e] * b[e];
  return ss;
}

__device__ __forceinline__ uint32_t half16(const uint4& r, int e) {
  const uint32_t w = e < 2 ? r.x : e < 4 ? r.y : e < 6 ? r.z : r.w;
  return (e & 1) ? (w >> 16) : (w & 0xffffu);
}

__device__ __forceinline__ f32x4 mfma_f32_16x16x4(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// D += X[16x16] Y[16x16] (fp32 MFMA); X row-major (stride xs); Y row-major, or column-major when yT.
__device__ __forceinline__ f32x4 mm16_f32(const float* X, int xs, const float* Y, int ys, bool yT, f32x4 acc,
                                          int lane) {
  const int i = lane & 15, kk = lane >> 4;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float yv = yT ? Y[i * ys + 4 * s + kk] : Y[(4 * s + kk) * ys + i];
    acc = mfma_f32_16x16x4(X[i * xs + 4 * s + kk], yv, acc);
  }
  return acc;
}

template <typename Tin>
__global__ __launch_bounds__(256, 2) void gdn_chunk_prep_kernel(const Tin* __restrict__ q, const Tin* __restrict__ k,
                                                                const Tin* __restrict__ v, const float* __restrict__ g,
                                                                const float* __restrict__ beta, ChunkWs ws, int T,
                                                                int NC, int Hk, int H, float scale, int l2norm) {
  __shared__ __attribute__((aligned(16))) __bf16 kt[kD * kC];     // raw k, transposed + swizzled
  __shared__ __attribute__((aligned(16))) __bf16 vt[kD * kC];     // raw v, transposed + swizzled
  __shared__ __attribute__((aligned(16))) float Am[kC * kFS];     // L; T' diag blocks; T_ij (i > j) at block (j, i)
  __shared__ __attribute__((aligned(16))) __bf16 pl[kC * kPS];    // P (bf16), lower triangle
  __shared__ __attribute__((aligned(16))) float scr[4][16 * 17];  // per-wave 16x16 scratch
  __shared__ float gam[kC], bet[kC], rkn[kC], rqn[kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int kh = h / (H / Hk);
  const int t0 = c * kC;
  const int nvalid = min(kC, T - t0);
  const size_t bhc = ((size_t)b * H + h) * NC + c;
  auto krow = [&](int row) { return k + (((size_t)b * T + t0 + row) * Hk + kh) * kD; };
  auto qrow = [&](int row) { return q + (((size_t)b * T + t0 + row) * Hk + kh) * kD; };

  // 1. stage: threads 0-127 transpose k (and take |k| per row), threads 128-255 transpose v and take |q| per row;
  //    unit = 8 rows x 8 dims. The last wave also forms the gates.
  {
    const int u = tid & 127, rg = u >> 4, cc = u & 15;
    const bool isK = tid < 128;
    uint4 raw[8], rq[8];
    const Tin* src[8];
    const Tin* qsrc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = min(8 * rg + i, nvalid - 1);
      const size_t tok = (size_t)b * T + t0 + row;
      src[i] = isK ? k + (tok * Hk + kh) * kD + 8 * cc : v + (tok * H + h) * kD + 8 * cc;
      qsrc[i] = q + (tok * Hk + kh) * kD + 8 * cc;
      raw[i] = raw8(src[i]);
    }
    if (!isK) {
#pragma unroll
      for (int i = 0; i < 8; ++i) rq[i] = raw8(qsrc[i]);
    }
    float ss[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool valid = 8 * rg + i < nvalid;
      ss[i] = valid ? (isK ? sumsq8_in(src[i], raw[i]) : sumsq8_in(qsrc[i], rq[i])) : 0.f;
      raw[i] = mask8(raw[i], valid);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) ss[i] += __shfl_xor(ss[i], off, 64);
    }
    if (cc == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) (isK ? rkn : rqn)[8 * rg + i] = l2norm ? rsqrtf(ss[i] + 1e-6f) : 1.f;
    }
    __bf16* dst = isK ? kt : vt;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = 8 * cc + e;
      uint4 w;
      w.x = half16(raw[0], e) | (half16(raw[1], e) << 16);
      w.y = half16(raw[2], e) | (half16(raw[3], e) << 16);
      w.z = half16(raw[4], e) | (half16(raw[5], e) << 16);
      w.w = half16(raw[6], e) | (half16(raw[7], e) << 16);
      *reinterpret_cast<uint4*>(dst + d * kC + 8 * (rg ^ swz(d))) = w;
    }
    if (wave == 3) {  // gates: gamma = cumsum(g), beta (zero in the padded tail, as HF pads g and beta with 0)
      float gv = 0.f, bv = 0.f;
      if (lane < nvalid) {
        const size_t idx = ((size_t)b * T + t0 + lane) * H + h;
        gv = g[idx];
        bv = beta[idx];
      }
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(gv, off, 64);
        if (lane >= off) gv += y;
      }
      gam[lane] = gv;
      bet[lane] = bv;
    }
  }
  __syncthreads();

  // 2. lower 16x16 tiles (mt >= nt) of K K^T and Q K^T from raw bf16 rows in L2 (all of the wave's operand loads
  //    issued before the first MFMA); l2norm / scale / decay applied in fp32.
  {
    const int np = wave < 2 ? 3 : 2;  // tiles p = wave, wave + 4, wave + 8 (< 10)
    bf16x8 opk[3][4], opq[3][4], opb[3][4];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int p = wave + 4 * i;
      const int mt = (p >= 1) + (p >= 3) + (p >= 6);
      const int nt = p - mt * (mt + 1) / 2;
      const int ra = 16 * mt + li, rb = 16 * nt + li;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int d0 = 32 * ks + 8 * lg;
        const int rac = min(ra, nvalid - 1), rbc = min(rb, nvalid - 1);
        const uint4 ka = mask8(raw8(krow(rac) + d0), ra < nvalid), qa = mask8(raw8(qrow(rac) + d0), ra < nvalid);
        const uint4 kb = mask8(raw8(krow(rbc) + d0), rb < nvalid);
        opk[i][ks] = *reinterpret_cast<const bf16x8*>(&ka);
        opq[i][ks] = *reinterpret_cast<const bf16x8*>(&qa);
        opb[i][ks] = *reinterpret_cast<const bf16x8*>(&kb);
      }
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i < np) {
        const int p = wave + 4 * i;
        const int mt = (p >= 1) + (p >= 3) + (p >= 6);
        const int nt = p - mt * (mt + 1) / 2;
        f32x4 ak = zero4(), aq = zero4();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          ak = mfma16(opk[i][ks], opb[i][ks], ak);
          aq = mfma16(opq[i][ks], opb[i][ks], aq);
        }
        const int s = 16 * nt + li;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * mt + 4 * lg + r;
          const float dec = s <= t ? __expf(gam[t] - gam[s]) : 0.f;
          const float kk = ak[r] * rkn[t] * rkn[s];
          const float qk = aq[r] * rqn[t] * scale * rkn[s];
          Am[t * kFS + s] = s < t ? -bet[t] * kk * dec : 0.f;
          pl[t * kPS + s] = (__bf16)(qk * dec);
        }
      }
    }
  }
  __syncthreads();

  // 3. diagonal 16x16 blocks: T' = strictly-lower part of (I - L_bb)^-1 by forward substitution in registers.
  //    Lane j keeps column j; row i's original entries are broadcast with readlane before row i is overwritten.
  {
    const int bb = wave;
    float tc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) tc[i] = Am[(16 * bb + i) * kFS + 16 * bb + li];
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      float acc = tc[i];
#pragma unroll
      for (int j = 0; j < i; ++j) {
        const float lij = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tc[i]), j));
        acc += lij * tc[j];
      }
      tc[i] = acc;
    }
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < 16; ++i) Am[(16 * bb + i) * kFS + 16 * bb + lane] = tc[i];
    }
  }
  __syncthreads();

  // 4. off-diagonal blocks T_ij = (I + T'_ii) sum_{k=j}^{i-1} L_ik T_kj with T_jj = I + T'_jj. Block column j depends
  //    only on its own earlier blocks, so wave j runs column j as an independent chain (no block barriers);
  //    T_ij is stored transposed in the unused upper block (j, i).
  {
    auto blk = [&](int bi, int bj) { return Am + (16 * bi) * kFS + 16 * bj; };
    const int j = wave;
    float* sc = scr[wave];
    for (int i = j + 1; i < 4; ++i) {
      f32x4 acc;
      const float* Lij = blk(i, j);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = Lij[(4 * lg + r) * kFS + li];
      acc = mm16_f32(Lij, kFS, blk(j, j), kFS, false, acc, lane);
      for (int kk = j + 1; kk < i; ++kk) acc = mm16_f32(blk(i, kk), kFS, blk(j, kk), kFS, true, acc, lane);
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[(4 * lg + r) * 17 + li] = acc[r];
      __builtin_amdgcn_wave_barrier();
      acc = mm16_f32(blk(i, i), kFS, sc, 17, false, acc, lane);
      // store transposed: element (row 4 lg + r, col li) of T_ij at block (j, i) [li][4 lg + r]
      *reinterpret_cast<f32x4*>(blk(j, i) + li * kFS + 4 * lg) = acc;
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();

  // 5a. outputs independent of T: K~^T, Q~, P, exp(gamma_last)
  const float gl = gam[kC - 1];
  {
    __bf16* KTo = ws.KT + bhc * kKTElems;
    // K~^T [mt 8][ks 2][lane][p] = k[s][d] rk_s exp(gl - gamma_s), s = 32 ks + kmap(lg, p), d = 16 mt + li
#pragma unroll
    for (int m2 = 0; m2 < 2; ++m2) {
      const int mt = 2 * wave + m2, d = 16 * mt + li;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int s0 = 32 * ks + 4 * lg, s1 = s0 + 16;
        const uint2 lo = *reinterpret_cast<const uint2*>(kt + tofs(d, s0));
        const uint2 hi = *reinterpret_cast<const uint2*>(kt + tofs(d, s1));
        const float x[8] = {bf16lo(lo.x), bf16hi(lo.x), bf16lo(lo.y), bf16hi(lo.y),
                            bf16lo(hi.x), bf16hi(hi.x), bf16lo(hi.y), bf16hi(hi.y)};
        bf16x8 o8;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const int s = p < 4 ? s0 + p : s1 + p - 4;
          o8[p] = (__bf16)(x[p] * rkn[s] * __expf(gl - gam[s]));
        }
        *reinterpret_cast<bf16x8*>(KTo + ((mt * 2 + ks) * 64 + lane) * 8) = o8;
      }
    }
    // Q~ [mt 4][ks 4][lane][p] = q[t][32 ks + kmap(lg, p)] rq_t scale exp(gamma_t), t = 16 mt + li
    {
      __bf16* Qo = ws.Q + bhc * kQElems;
      const int mt = wave, t = 16 * mt + li;
      const float f = rqn[t] * scale * __expf(gam[t]);
      const Tin* qr = qrow(min(t, nvalid - 1));
      f32x4 lo[4], hi[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        lo[ks] = load4f(qr + 32 * ks + 4 * lg);
        hi[ks] = load4f(qr + 32 * ks + 16 + 4 * lg);
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        bf16x8 o8;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o8[e] = (__bf16)(t < nvalid ? lo[ks][e] * f : 0.f);
          o8[4 + e] = (__bf16)(t < nvalid ? hi[ks][e] * f : 0.f);
        }
        *reinterpret_cast<bf16x8*>(Qo + ((mt * 4 + ks) * 64 + lane) * 8) = o8;
      }
    }
    // P [mt 4][ks 2][lane][p] = P[16 mt + li][32 ks + kmap(lg, p)] (zero above the diagonal)
    {
      __bf16* Po = ws.P + bhc * kPElems;
      const int mt = wave, t = 16 * mt + li;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        bf16x8 o8;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const int s = 32 * ks + kmap(lg, p);
          o8[p] = s <= t ? pl[t * kPS + s] : (__bf16)0.f;
        }
        *reinterpret_cast<bf16x8*>(Po + ((mt * 2 + ks) * 64 + lane) * 8) = o8;
      }
    }
    if (tid < 64) {
      const float e = __expf(gl);
      const f32x4 e4 = {e, e, e, e};
      *reinterpret_cast<f32x4*>(ws.EG + bhc * kEGElems + 4 * tid) = e4;
    }
  }

  // 5b. A operands of U = T diag(beta) V and W = T diag(beta exp(gamma) rk) K from the assembled T
  const int mt = wave, t = 16 * mt + li;
  bf16x8 au[2], aw[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int s = 32 * ks + 8 * lg + jj;
      const int bs = s >> 4;
      float tv;
      if (bs == mt) tv = (t == s ? 1.f : 0.f) + (s < t ? Am[t * kFS + s] : 0.f);
      else if (bs < mt) tv = Am[s * kFS + t];  // T_{mt, bs} stored transposed at block (bs, mt)
      else tv = 0.f;
      tv *= bet[s];
      au[ks][jj] = (__bf16)tv;
      aw[ks][jj] = (__bf16)(tv * __expf(gam[s]) * rkn[s]);
    }
  }
  __syncthreads();  // every wave has read Am; it becomes the W staging array

  // 5c. U (fp32, scan-kernel accumulator order) and W (bf16, staged for the swizzled store)
  {
    float* Uo = ws.U + bhc * kUElems;
    __bf16* wl = reinterpret_cast<__bf16*>(Am);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int d = 16 * nt + li;
      f32x4 accu = zero4(), accw = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int pos = 32 * ks + 8 * lg;
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(vt + tofs(d, pos));
        const bf16x8 bk = *reinterpret_cast<const bf16x8*>(kt + tofs(d, pos));
        accu = mfma16(au[ks], bv, accu);
        accw = mfma16(aw[ks], bk, accw);
      }
      *reinterpret_cast<f32x4*>(Uo + ((nt * 4 + mt) * 64 + lane) * 4) = accu;
#pragma unroll
      for (int r = 0; r < 4; ++r) wl[(16 * mt + 4 * lg + r) * kWS + d] = (__bf16)accw[r];
    }
  }
  __syncthreads();
  {
    __bf16* Wo = ws.W + bhc * kWElems;
    const __bf16* wl = reinterpret_cast<const __bf16*>(Am);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const uint2 lo = *reinterpret_cast<const uint2*>(wl + t * kWS + 32 * ks + 4 * lg);
      const uint2 hi = *reinterpret_cast<const uint2*>(wl + t * kWS + 32 * ks + 16 + 4 * lg);
      uint4 o;
      o.x = lo.x; o.y = lo.y; o.z = hi.x; o.w = hi.y;
      *reinterpret_cast<uint4*>(Wo + ((mt * 4 + ks) * 64 + lane) * 8) = o;
    }
  }
}

// Hand-over slot from the recurrence wave to the output wave: packed state (4 B operands) and packed Vn (2).
struct ScanSlot {
  bf16x8 sb[4][64];
  bf16x8 vb[2][64];
};
// LDS prefetch stages, filled by global_load_lds_dwordx4 (lane i's 16 bytes land at +16 i of each 1 KB record):
// the recurrence wave's W, K~^T and own U slice; the output wave's Q~ and P.
struct RecStage {
  bf16x8 w[16][64];
  bf16x8 kt[16][64];
  f32x4 u[4][64];
  f32x4 eg[64];
};
struct OutStage {
  bf16x8 q[16][64];
  bf16x8 p[8][64];
};

// Copy n consecutive 1 KB records (src, 64 lanes x 16 B each) into LDS records (dst) without touching registers:
// one global_load_lds_dwordx4 per record, M0 = LDS destination. The instructions are issued from inline asm so that
// the compiler does not track them as LDS writes (its tracking would make every later LDS read wait for all of
// them); the kernels order them with explicit vmcnt waits instead.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma_records(const void* src, void* dst, int n, int lane) {
  const char* s = reinterpret_cast<const char*>(src) + lane * 16;
  const uint32_t d = lds_addr(dst);
#pragma unroll
  for (int i = 0; i < n; ++i)
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(d + i * 1024), "v"(s + i * 1024)
                 : "memory", "m0");
}

// Blocks are dispatched round-robin over the 8 XCDs (block i runs on XCD i % 8). The 8 column slices of one
// (row, head) read the same W / K~^T / Q~ / P records, so they are mapped onto one XCD to share its L2: block L
// serves XCD x = L % 8, and the j-th block of that XCD (j = L / 8) is slice j % 8 of head-row unit 8 (j / 8) + x.
// When the number of (row, head) units is not a multiple of 8 the plain slice-fastest mapping is used.
__device__ __forceinline__ void scan_block_coords(int L, int nunits, int& sl, int& unit) {
  if ((nunits & 7) == 0) {
    const int x = L & 7, j = L >> 3;
    sl = j & 7;
    unit = 8 * (j >> 3) + x;
  } else {
    sl = L & 7;
    unit = L >> 3;
  }
}

__device__ __forceinline__ void store_out(__amdgpu_buffer_rsrc_t rc, int off_elems, float x, __bf16*) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (__bf16)x), rc, off_elems * 2, 0, 0);
}
__device__ __forceinline__ void store_out(__amdgpu_buffer_rsrc_t rc, int off_elems, float x, float*) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, x), rc, off_elems * 4, 0, 0);
}

// Number of vector-memory operations the output wave issues per chunk besides its prefetch: one store per output.
constexpr int kOutStores = 16;

template <typename Tin>
__global__ __launch_bounds__(128) void gdn_chunk_scan_kernel(ChunkWs ws, const float* s_in, float* s_out,
                                                             Tin* __restrict__ o, int T, int NC, int H, int B) {
  __shared__ ScanSlot slot[2];
  __shared__ RecStage rst[2];
  __shared__ OutStage ost[2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sl, unit;
  scan_block_coords(blockIdx.x, H * B, sl, unit);
  const int h = unit % H, b = unit / H;
  const int li = lane & 15, lg = lane >> 4;
  const int col = 16 * sl + li;
  const size_t bh = (size_t)b * H + h;

  if (wave == 0) {
    // ---------------- recurrence wave ----------------
    const size_t sbase = bh * kD * kD;
    f32x4 S[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[mt][r] = s_in ? s_in[sbase + (size_t)(16 * mt + 4 * lg + r) * kD + col] : 0.f;
    auto prefetch = [&](int c, RecStage& st) {
      const size_t bhc = bh * NC + c;
      dma_records(ws.W + bhc * kWElems, &st.w[0][0], 16, lane);
      dma_records(ws.KT + bhc * kKTElems, &st.kt[0][0], 16, lane);
      dma_records(ws.U + bhc * kUElems + (size_t)sl * 4 * 64 * 4, &st.u[0][0], 4, lane);
      dma_records(ws.EG + bhc * kEGElems, &st.eg[0], 1, lane);
    };
    prefetch(0, rst[0]);
    for (int c = 0; c < NC; ++c) {
      // issue the next chunk's 37 records (the last chunk re-reads itself: no branch), then wait for this chunk's,
      // which were issued one iteration earlier
      const int cn = c + 1 < NC ? c + 1 : c;
      prefetch(cn, rst[(c + 1) & 1]);
      asm volatile("s_waitcnt vmcnt(37)" ::: "memory");
      const RecStage& st = rst[c & 1];
      const float eg = st.eg[lane][0];
      ScanSlot& sd = slot[c & 1];
      bf16x8 sb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        sb[ks] = pack8(S[2 * ks], S[2 * ks + 1]);
        sd.sb[ks][lane] = sb[ks];
      }
      f32x4 vn[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) acc = mfma16(st.w[mt * 4 + ks][lane], sb[ks], acc);
        const f32x4 u = st.u[mt][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) vn[mt][r] = u[r] - acc[r];
      }
      bf16x8 vb[2];
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        vb[k2] = pack8(vn[2 * k2], vn[2 * k2 + 1]);
        sd.vb[k2][lane] = vb[k2];
      }
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) S[mt][r] *= eg;
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) S[mt] = mfma16(st.kt[mt * 2 + k2][lane], vb[k2], S[mt]);
      }
      lds_barrier();  // slot c & 1 is complete (the next chunk's records stay in flight)
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // drain the last (redundant) prefetch before LDS goes away
    if (s_out) {
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_out[sbase + (size_t)(16 * mt + 4 * lg + r) * kD + col] = S[mt][r];
    }
  } else {
    // ---------------- output wave ----------------
    // Outputs go through a buffer resource spanning row b's [T, H, 128] block: stores past the sequence end fall
    // outside it and are dropped by the hardware, so the store path has no branch.
    const __amdgpu_buffer_rsrc_t orc = __builtin_amdgcn_make_buffer_rsrc(
        o + (size_t)b * T * H * kD, 0, (int)((size_t)T * H * kD * sizeof(Tin)), 0x00020000);
    auto prefetch = [&](int c, OutStage& st) {
      const size_t bhc = bh * NC + c;
      dma_records(ws.Q + bhc * kQElems, &st.q[0][0], 16, lane);
      dma_records(ws.P + bhc * kPElems, &st.p[0][0], 8, lane);
    };
    prefetch(0, ost[0]);
    for (int c = 0; c < NC; ++c) {
      const int cn = c + 1 < NC ? c + 1 : c;
      prefetch(cn, ost[(c + 1) & 1]);
      // this chunk's 24 records are older than the 24 just issued and the previous chunk's stores
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(24 + kOutStores) : "memory");
      lds_barrier();  // the recurrence wave has filled slot c & 1
      const OutStage& st = ost[c & 1];
      const ScanSlot& sd = slot[c & 1];
      bf16x8 sb[4], vb[2];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) sb[ks] = sd.sb[ks][lane];
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) vb[k2] = sd.vb[k2][lane];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) acc = mfma16(st.q[mt * 4 + ks][lane], sb[ks], acc);
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) acc = mfma16(st.p[mt * 2 + k2][lane], vb[k2], acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = c * kC + 16 * mt + 4 * lg + r;
          store_out(orc, (t * H + h) * kD + col, acc[r], (Tin*)nullptr);
        }
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

}  // namespace q35

extern "C" size_t q35_gdn_chunk_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t Dk, int64_t Dv,
                                                int64_t chunk_size) {
  using namespace q35;
  if (B <= 0 || T <= 0 || H <= 0 || Dk != kD || Dv != kD || chunk_size != kC) return 0;
  const size_t NC = (size_t)((T + kC - 1) / kC);
  size_t total = 0;
  chunk_ws_layout(nullptr, (size_t)B * H * NC, &total);
  return total;
}

extern "C" int q35_gdn_chunk_prefill(const void* q, const void* k, const void* v, const float* g, const float* beta,
                                     const float* initial_state, float* final_state, void* out, int64_t B, int64_t T,
                                     int64_t Hk, int64_t H, int64_t Dk, int64_t Dv, int dtype, float scale,
                                     int use_qk_l2norm, int64_t chunk_size, void* workspace, size_t workspace_bytes,
                                     q35_stream_t stream) {
  using namespace q35;
  if (!q || !k || !v || !g || !beta || !out) return Q35_EINVAL;
  if (B <= 0 || T <= 0 || Hk <= 0 || H <= 0 || Dk <= 0 || Dv <= 0 || H % Hk != 0 || chunk_size <= 0)
    return Q35_EINVAL;
  if (Dk != kD || Dv != kD || chunk_size != kC) return Q35_EUNSUPPORTED;
  if (B > 65535 || H > 65535 || H * B > (1 << 27) || T > ((int64_t)1 << 30) / (H > Hk ? H : Hk))
    return Q35_EUNSUPPORTED;
  // the output buffer resource spans one row's [T, H, 128] block and is addressed with 32-bit byte offsets
  if (T * H * kD * (dtype == Q35_F32 ? 4 : 2) >= ((int64_t)1 << 31)) return Q35_EUNSUPPORTED;
  if (dtype != Q35_F32 && dtype != Q35_BF16) return Q35_EUNSUPPORTED;
  const int64_t NC = (T + kC - 1) / kC;
  if (NC > 0x7fffffff) return Q35_EUNSUPPORTED;
  size_t need = 0;
  ChunkWs ws = chunk_ws_layout(workspace, (size_t)B * H * NC, &need);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255)) return Q35_EWORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 g1((unsigned)NC, (unsigned)H, (unsigned)B), g2((unsigned)(kD / 16 * H * B));
  if (dtype == Q35_F32) {
    hipLaunchKernelGGL(gdn_chunk_prep_kernel<float>, g1, dim3(256), 0, st, (const float*)q, (const float*)k,
                       (const float*)v, g, beta, ws, (int)T, (int)NC, (int)Hk, (int)H, scale, use_qk_l2norm);
    hipLaunchKernelGGL(gdn_chunk_scan_kernel<float>, g2, dim3(128), 0, st, ws, initial_state, final_state,
                       (float*)out, (int)T, (int)NC, (int)H, (int)B);
  } else {
    hipLaunchKernelGGL(gdn_chunk_prep_kernel<__bf16>, g1, dim3(256), 0, st, (const __bf16*)q, (const __bf16*)k,
                       (const __bf16*)v, g, beta, ws, (int)T, (int)NC, (int)Hk, (int)H, scale, use_qk_l2norm);
    hipLaunchKernelGGL(gdn_chunk_scan_kernel<__bf16>, g2, dim3(128), 0, st, ws, initial_state, final_state,
                       (__bf16*)out, (int)T, (int)NC, (int)H, (int)B);
  }
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
