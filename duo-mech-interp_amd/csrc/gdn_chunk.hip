// Gated DeltaNet, chunked form (prefill): chunk-64 UT/WY transform, fp32 state carried across the sequence.
// Two kernel pairs, chosen by the input dtype: bf16 q/k/v run the pair-record kernels below (bf16 MFMA products,
// fp32 accumulation); fp32 q/k/v run the fp32 WY kernels at the end of this file (every product in fp32).
//
// Math (HF:249-327 torch_chunk_gated_delta_rule; decay masks and the 63-row forward substitution at HF:288-298).
// Per (b, h), with q^ = l2norm(q) * scale, k^ = l2norm(k) and, inside a span of positions, gamma = cumsum(g):
//   L[t][s] = -beta_t (k^_t . k^_s) exp(gamma_t - gamma_s)  (s < t),     T = (I - L)^-1
//   U = T diag(beta) V,   W = T diag(beta exp(gamma)) K^,   P[t][s] = (q^_t . k^_s) exp(gamma_t - gamma_s)  (s <= t)
//   per span:  O = (Q^ exp(gamma)) S + P (U - W S),   S <- exp(gamma_last) S + K~^T (U - W S),
//              K~[s] = k^_s exp(gamma_last - gamma_s).
// Every exponent is <= 0 (g <= 0), so nothing overflows. HF applies this per chunk of 64; two consecutive chunks are
// one span of 128 here: T of the pair is block lower-triangular with the two chunk-64 inverses T00, T11 on its
// diagonal and T10 = T11 L10 T00 below, so W and U of the pair are the chunk-64 ones with the second chunk's
// corrected by the first's:  W1 = T11 (K'1 + L10 W0),  U1 = T11 (V'1 + L10 U0).
//
// The serial part is regrouped so that one scan step (one pair) is a single matrix product on the state:
//   S <- exp(G) S + M S + Bm,    O = Q' S + R,   with  M = -K~^T W,  Bm = K~^T U,  Q' = Q^ exp(gamma) - P W,  R = P U
// (exact algebra: U - W S substituted into both lines). M, Bm, Q', R depend on the inputs only, so all of them come
// out of one fully parallel kernel, and the sequential kernel streams 128 x 128 bf16 matrices per 128 positions.
//
// Kernel 1, gdn_pair_prep4_kernel: one block of 4 waves per (pair, head, row), all pairs in parallel, two blocks per
// compute unit. k, q, v rows are staged in padded LDS tiles (row-major for the K K^T / Q K^T products, transposed for
// the products that contract over positions); the two 64 x 64 inverses run in fp32 (16 x 16 diagonal blocks by
// forward substitution, off-diagonal blocks by per-column chains on fp32 MFMA); every other product is bf16 MFMA with
// fp32 accumulation. The products are oriented so that their accumulator tiles pack straight into the scan kernel's
// MFMA operand order, and the records are written with 16- or 8-byte coalesced stores.
// Kernel 2, gdn_pair_scan_kernel: 16 blocks per (row, head): 8 slices of 16 value columns x 2 halves of the output
// rows. Each block carries its 128 x 16 fp32 state slice in registers (8 waves x 16 rows) while 4 more waves form the
// 64 output rows of its half, 4 MFMAs per wave and pair (computed transposed, so that a lane holds 4 consecutive
// value columns of one position and writes them with one 8-byte store); the bf16 state is exchanged through LDS once
// per pair.
// Operands stream straight from L2 into registers three pairs ahead (12 waves keep about 40 KB of loads in flight per
// CU). The 16 blocks of a head are placed on one XCD (they share its L2). Each pair costs about 0.9 us: the state
// update's LDS exchange, barrier and 4 dependent MFMAs take about 0.3 us, and the rest follows the 54 KB of operands
// each compute unit streams per pair (M alone is 32 KB, needed whole by every slice).
#include <type_traits>

#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kC = 64;        // chunk of the UT transform
constexpr int kP = 128;       // positions per scan step (two chunks)
constexpr int kD = 128;       // Dk = Dv
constexpr int kFS = kC + 4;   // row stride (floats) of the fp32 64 x 64 inversion arrays

// Record of one (b, h, pair), bytes. Fragment order: [row tile][k step][lane][8] bf16, lane l holding row
// 16 rt + l % 16 and columns 32 ks + kmap(l / 16, j) (kmap below); D order: [row tile][slice][lane][4] bf16, lane l
// holding rows 16 rt + 4 (l / 16) + r of column 16 slice + l % 16 (the MFMA accumulator layout); transposed D order:
// the same tiles with lane l holding row 16 rt + l % 16 and columns 16 slice + 4 (l / 16) + r.
constexpr size_t kRecM = 0;           // M  = -K~^T W   [128 d][128 d]   fragment order
constexpr size_t kRecQ = 32768;       // Q'             [128 pos][128 d] fragment order
constexpr size_t kRecB = 65536;       // Bm = K~^T U    [128 d][128 dv]  D order
constexpr size_t kRecR = 98304;       // R  = P U       [128 pos][128 dv] transposed D order
constexpr size_t kRecE = 131072;      // exp(gamma_last) fp32
constexpr size_t kRecBytes = 131328;  // 256-byte aligned

constexpr int kScanAhead = 3;    // pairs whose operands are held in registers ahead of use

// k index of position j (0..7) of lane group g in a 32-wide K step fed from two 16-row accumulator tiles
__device__ __forceinline__ int kmap(int g, int j) { return j < 4 ? 4 * g + j : 12 + 4 * g + j; }

// Raw loads as packed bf16 bits, issued unconditionally from clamped addresses; rows outside the sequence are
// zeroed afterwards with a select.
__device__ __forceinline__ u32x4 raw8(const __bf16* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ f32x4 unpack_bf16x4(const u32x2& r) {
  f32x4 o = {bf16lo(r.x), bf16hi(r.x), bf16lo(r.y), bf16hi(r.y)};
  return o;
}
// Four consecutive bf16 inputs as loaded, converted to fp32 only when used: a raw load can be issued long before its
// use while holding half the registers.
struct Raw4 {
  u32x2 r;
  __device__ __forceinline__ void load(const __bf16* p) { r = *reinterpret_cast<const u32x2*>(p); }
  __device__ __forceinline__ f32x4 f() const { return unpack_bf16x4(r); }
};
__device__ __forceinline__ u32x4 mask8(u32x4 r, bool keep) {
  const u32x4 z = {0u, 0u, 0u, 0u};
  return keep ? r : z;
}
__device__ __forceinline__ float sumsq8(const u32x4& r) {
  const float x[8] = {bf16lo(r.x), bf16hi(r.x), bf16lo(r.y), bf16hi(r.y),
                      bf16lo(r.z), bf16hi(r.z), bf16lo(r.w), bf16hi(r.w)};
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  return ss;
}
__device__ __forceinline__ uint32_t half16(const u32x4& r, int e) {
  const uint32_t w = e < 2 ? r.x : e < 4 ? r.y : e < 6 ? r.z : r.w;
  return (e & 1) ? (w >> 16) : (w & 0xffffu);
}
// 8x8 bf16 transpose: column e of 8 rows (one 16-byte row segment each) as one 16-byte segment
__device__ __forceinline__ u32x4 column8(const u32x4 (&raw)[8], int e) {
  u32x4 w;
  w.x = half16(raw[0], e) | (half16(raw[1], e) << 16);
  w.y = half16(raw[2], e) | (half16(raw[3], e) << 16);
  w.z = half16(raw[4], e) | (half16(raw[5], e) << 16);
  w.w = half16(raw[6], e) | (half16(raw[7], e) << 16);
  return w;
}
__device__ __forceinline__ u32x2 pack4(float a, float b, float c, float d) {
  bf16x4 r = {(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
  return __builtin_bit_cast(u32x2, r);
}
__device__ __forceinline__ f32x4 unpack4(const u32x2& r) {
  f32x4 o = {bf16lo(r.x), bf16hi(r.x), bf16lo(r.y), bf16hi(r.y)};
  return o;
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

// First fragment of row tile rt in the packed lower-triangular P store (row tile rt has rt / 2 + 1 k steps).
__device__ __forceinline__ int pbase(int rt) { return (rt >> 1) * ((rt >> 1) + 1) + (rt & 1) * ((rt >> 1) + 1); }
constexpr int kPFrags = 20;

// Unit lower-triangular 64 x 64 inverse in place (fp32, row stride kFS): on entry the strictly-lower part of `Am`
// holds L (zeros on and above the diagonal of the diagonal blocks); on exit block (i, i) holds the strictly-lower
// part of its diagonal inverse and, for i > j, T_ij is stored transposed in the unused upper block (j, i). Four
// waves: wave bb inverts diagonal block bb, then runs block column bb. `bar` is a barrier of all waves of the block.
template <typename Bar>
__device__ __forceinline__ void invert64(float* Am, int bb, int lane, float* sc, Bar bar) {
  const int li = lane & 15, lg = lane >> 4;
  {
    // forward substitution: lane j keeps column j; row i's original entries are broadcast with readlane before row i
    // is overwritten
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
  bar();
  // T_ij = (I + T'_ii) sum_{k=j}^{i-1} L_ik T_kj with T_jj = I + T'_jj: column j is an independent chain
  auto blk = [&](int bi, int bj) { return Am + (16 * bi) * kFS + 16 * bj; };
  const int j = bb;
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
    *reinterpret_cast<f32x4*>(blk(j, i) + li * kFS + 4 * lg) = acc;
    __builtin_amdgcn_wave_barrier();
  }
}

// T[t][s] of a 64 x 64 inverse stored by invert64 (t, s in 0..63)
__device__ __forceinline__ float tinv(const float* Am, int t, int s) {
  const int bt = t >> 4, bs = s >> 4;
  if (bs == bt) return (t == s ? 1.f : 0.f) + (s < t ? Am[t * kFS + s] : 0.f);
  if (bs < bt) return Am[s * kFS + t];
  return 0.f;
}

// ---------------------------------------------------------------------------------------------------------------
// gdn_pair_prep4_kernel: the records of one (pair, head, row) from a 4-wave block with at most 80 KB of LDS and 256
// VGPRs, so that two blocks share a compute unit and every block of a T = 4096, 16-head call is resident at once (one
// block's memory and barrier waits are covered by the other's work).
//
// Dataflow. Waves 0-1 ("W waves") own value tiles D0 .. D0 + 3 (D0 = 4 (w & 1)) of W; waves 2-3 ("U waves") the same
// tiles of U. Each wave forms its tiles for all 128 positions (W0 = T00 K'0, Z = L10 W0 + K'1, W1 = T11 Z; U alike),
// keeps them in registers as MFMA operands (a D-layout accumulator tile is one half of a 32-wide k step: the kmap
// order) and from them writes its part of the records: M^T = -W^T K~ and Q'^T = Q^ e^gamma - W^T P^T (W waves),
// Bm = K~^T U and R^T = U^T P^T (U waves). LDS holds the row-major k tile (K K^T / Q K^T), then the two fp32 64 x 64
// L blocks (inverted in place), then V^T, then P; K^T stays for the whole block. Tiles are [128][128] bf16 with
// 272-byte rows: 16 lanes reading 16 consecutive rows at one column hit 16 distinct bank quads, and fragment
// addresses are a per-lane row base plus immediate offsets.
//
// Decay factors exp(gamma_t - gamma_s) (s < t): exact per element on diagonal 16 x 16 tiles; on tiles below the
// diagonal the product of a row factor exp(gamma_t - gamma_r) and a column factor exp(gamma_r - gamma_s) around the
// tile's first row r, both <= 1 (gamma is non-increasing), so neither overflows whatever the size of g.
constexpr int kRS = 272;  // bytes per row of a padded [128][128] bf16 LDS tile

__device__ __forceinline__ bf16x8 ldf(const char* tile, int r, int c) {  // row r, columns c .. c + 7
  return *reinterpret_cast<const bf16x8*>(tile + r * kRS + 2 * c);
}
// The transposed tiles (K^T, V^T: rows d, columns positions) swap 16-byte column chunks by row group: chunk j of
// row r is stored at chunk j ^ ((r / 16) % 8). A transposed write of 16 rows 8 apart then covers every bank once, while
// the fragment reads (16 consecutive rows of one group at one column) stay conflict-free.
__device__ __forceinline__ int tsw(int rg, int c) {  // byte offset of column c in a row of row group rg
  return 16 * ((c >> 3) ^ (rg & 7)) + 2 * (c & 7);
}
__device__ __forceinline__ bf16x8 ldf_t(const char* tile, int rg, int li, int c) {  // row 16 rg + li, columns c .. + 7
  return *reinterpret_cast<const bf16x8*>(tile + (16 * rg + li) * kRS + tsw(rg, c));
}
// row 16 rg + li, the 8 columns of k step c0 held by lane group g in kmap order: c0 + 4 g .. + 3, c0 + 16 + 4 g .. + 3
__device__ __forceinline__ bf16x8 ldf_km_t(const char* tile, int rg, int li, int c0, int g) {
  const char* row = tile + (16 * rg + li) * kRS;
  const u32x2 a = *reinterpret_cast<const u32x2*>(row + tsw(rg, c0 + 4 * g));
  const u32x2 b = *reinterpret_cast<const u32x2*>(row + tsw(rg, c0 + 16 + 4 * g));
  const u32x4 v = {a.x, a.y, b.x, b.y};
  return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ f32x4 scale4(const f32x4& a, const f32x4& s) {
  f32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = a[i] * s[i];
  return r;
}

// Inverses T = (I - L)^-1 of the two unit lower-triangular 64 x 64 blocks of a pair, in place in Am (two [64][kFS]
// fp32 arrays, strictly-lower L on entry with zeros on and above the diagonal of the diagonal 16 x 16 blocks; on exit
// T row-major with the strictly-lower part of its diagonal blocks stored and the unit diagonal implicit). Waves 2 m and
// 2 m + 1 take matrix m. With T_ii = I + T'_ii the diagonal inverses (forward substitution, wave w the blocks c and
// 3 - c, c = w % 2), the blocks below the diagonal follow from T_ij = T_ii sum_{k=j}^{i-1} L_ik T_kj in two levels of
// 2 x 2 block inversion:
//   level 1 (32 x 32 diagonal halves):  T_10 = T_11 L_10 T_00 (wave 2 m),  T_32 = T_33 L_32 T_22 (wave 2 m + 1)
//   level 2 (block column j = w % 2):    X_2j = L_20 T_0j + L_21 T_1j,  X_3j = L_30 T_0j + L_31 T_1j,
//                                        T_2j = T_22 X_2j,  T_3j = T_33 X_3j + T_32 X_2j
// Operands that a product takes as its B side are also stored transposed in the free blocks above the diagonal.
__device__ __forceinline__ void invert64x2(float* Am2, int wv, int lane) {
  const int li = lane & 15, lg = lane >> 4;
  float* Am = Am2 + (wv >> 1) * 64 * kFS;
  const int c0 = wv & 1, c1 = 3 - c0;
  auto blk = [&](int bi, int bj) { return Am + (16 * bi) * kFS + 16 * bj; };
  {
    // lane groups 0-1 take diagonal block c0, groups 2-3 block c1 (groups 1 and 3 repeat 0 and 2); lane li keeps
    // column li, T'[i][li] = L[i][li] + sum_{j < i} L[i][j] T'[j][li], with row i of L read from LDS as a broadcast
    // (LDS keeps L until the end)
    // (the scheduling barriers keep the compiler from hoisting every row's reads at once, which would hold 60 more
    // registers at the kernel's register limit)
    float* Dg = lg < 2 ? blk(c0, c0) : blk(c1, c1);
    float tc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) tc[i] = Dg[i * kFS + li];
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      f32x4 lr[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (4 * q < i) lr[q] = *reinterpret_cast<const f32x4*>(Dg + i * kFS + 4 * q);
      float acc = tc[i];
#pragma unroll
      for (int j = 0; j < i; ++j) acc += lr[j >> 2][j & 3] * tc[j];
      tc[i] = acc;
      __builtin_amdgcn_sched_barrier(0);
    }
    if ((lg & 1) == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) Dg[i * kFS + li] = tc[i];
    }
  }
  lds_barrier();  // the diagonal blocks are inverted
  const bool wa = (wv & 1) == 0;
  auto ld_d = [&](const float* b) {  // a 16 x 16 block in the accumulator layout
    f32x4 v;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = b[(4 * lg + r) * kFS + li];
    return v;
  };
  auto st_d = [&](float* b, const f32x4& v) {
#pragma unroll
    for (int r = 0; r < 4; ++r) b[(4 * lg + r) * kFS + li] = v[r];
  };
  auto st_t = [&](float* b, const f32x4& v) { *reinterpret_cast<f32x4*>(b + li * kFS + 4 * lg) = v; };
  {
    // level 1: T_hl = (I + T'_hh) (L_hl + L_hl T'_ll), (h, l) = (1, 0) or (3, 2); L_hl is read by this wave only
    const int l = wa ? 0 : 2, h = l + 1;
    f32x4 acc = mm16_f32(blk(h, l), kFS, blk(l, l), kFS, false, ld_d(blk(h, l)), lane);
    st_t(blk(l, h), acc);
    __builtin_amdgcn_wave_barrier();
    acc = mm16_f32(blk(h, h), kFS, blk(l, h), kFS, true, acc, lane);
    __builtin_amdgcn_wave_barrier();
    st_d(blk(h, l), acc);
    st_t(blk(l, h), acc);
  }
  lds_barrier();  // T_10 (also transposed in block (0, 1)) and T_32 are in place
  {
    const int j = wa ? 0 : 1;
    f32x4 x2 = mm16_f32(blk(2, j), kFS, blk(j, j), kFS, false, ld_d(blk(2, j)), lane);
    f32x4 x3 = mm16_f32(blk(3, j), kFS, blk(j, j), kFS, false, ld_d(blk(3, j)), lane);
    if (wa) {  // column 0 also takes L_21 T_10, L_31 T_10
      x2 = mm16_f32(blk(2, 1), kFS, blk(0, 1), kFS, true, x2, lane);
      x3 = mm16_f32(blk(3, 1), kFS, blk(0, 1), kFS, true, x3, lane);
    }
    st_t(blk(j, 2), x2);
    st_t(blk(j, 3), x3);
    __builtin_amdgcn_wave_barrier();
    const f32x4 t2 = mm16_f32(blk(2, 2), kFS, blk(j, 2), kFS, true, x2, lane);
    f32x4 t3 = mm16_f32(blk(3, 3), kFS, blk(j, 3), kFS, true, x3, lane);
    t3 = mm16_f32(blk(3, 2), kFS, blk(j, 2), kFS, true, t3, lane);
    lds_barrier();  // every L block below the diagonal is read
    st_d(blk(2, j), t2);
    st_d(blk(3, j), t3);
  }
}

__global__ __launch_bounds__(256, 2) void gdn_pair_prep4_kernel(const __bf16* __restrict__ q,
                                                                const __bf16* __restrict__ k,
                                                                const __bf16* __restrict__ v,
                                                                const float* __restrict__ g,
                                                                const float* __restrict__ beta, char* __restrict__ ws,
                                                                int T, int NP, int Hk, int H, float scale,
                                                                int l2norm) {
  __shared__ __attribute__((aligned(16))) char RA[kP * kRS];  // k rows -> L00, L11 fp32 -> T -> V^T -> P fragments
  __shared__ __attribute__((aligned(16))) char RB[kP * kRS];  // K^T [d][pos]
  __shared__ __attribute__((aligned(16))) bf16x8 L10f[8][64];  // L10 A fragments [c1 row tile][k step], kmap order
  // per position: 0 gamma; 1 beta; 2 rk, then rk e^(gamma_last - gamma) (K~); 3 rq scale, then rq scale e^gamma
  // (Q^ e^gamma, 0 past the end); 4 beta e^gamma rk (W's input scale)
  __shared__ __attribute__((aligned(16))) float cf[5][kP];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int h = blockIdx.x, p = blockIdx.y, b = blockIdx.z;
  const int kh = h / (H / Hk);
  const int t0 = p * kP;
  const int nvalid = min(kP, T - t0);
  char* rec = ws + (((size_t)b * H + h) * NP + p) * kRecBytes;
  float* Am = reinterpret_cast<float*>(RA);

  // ---- 0. stage: each thread an 8 x 8 unit of k (positions 8 ur .., dims 8 uc ..) into the row-major tile (RA) and
  //         transposed into K^T (RB); the wave's own q rows (row tiles X0 = w, X1 = 7 - w) as B fragments in
  //         registers; the gates (wave 0). Every load goes out before any is used.
  const int ur = tid >> 4, uc = tid & 15;
  // per-block bases (64-bit, uniform) and 32-bit offsets inside the pair (T H 128 < 2^31 is checked by the launcher)
  const __bf16* kb = k + (((size_t)b * T + t0) * Hk + kh) * kD;
  const __bf16* qb = q + (((size_t)b * T + t0) * Hk + kh) * kD;
  const __bf16* vb = v + (((size_t)b * T + t0) * H + h) * kD;
  const int kstride = Hk * kD, vstride = H * kD;
  u32x4 raw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) raw[i] = raw8(kb + min(8 * ur + i, nvalid - 1) * kstride + 8 * uc);
  const int X0 = wv, X1 = 7 - wv;
  bf16x8 qf[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int t = 16 * (a ? X1 : X0) + li;
    const __bf16* src = qb + min(t, nvalid - 1) * kstride;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[a][ks] = *reinterpret_cast<const bf16x8*>(src + 32 * ks + 8 * lg);
  }
  float g0 = 0.f, g1 = 0.f, b0 = 0.f, b1 = 0.f;
  if (wv == 0) {
    const size_t base = ((size_t)b * T + t0) * H + h;
    if (lane < nvalid) { g0 = g[base + (size_t)lane * H]; b0 = beta[base + (size_t)lane * H]; }
    if (64 + lane < nvalid) { g1 = g[base + (size_t)(64 + lane) * H]; b1 = beta[base + (size_t)(64 + lane) * H]; }
  }
  {
    float ss[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool valid = 8 * ur + i < nvalid;
      ss[i] = valid ? sumsq8(raw[i]) : 0.f;
      raw[i] = mask8(raw[i], valid);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) ss[i] += __shfl_xor(ss[i], off, 64);
    }
    if (uc == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) cf[2][8 * ur + i] = l2norm ? rsqrtf(ss[i] + 1e-6f) : 1.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4*>(RA + (8 * ur + i) * kRS + 16 * uc) = raw[i];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      *reinterpret_cast<u32x4*>(RB + (8 * uc + e) * kRS + 16 * (ur ^ ((uc >> 1) & 7))) = column8(raw, e);
  }
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int t = 16 * (a ? X1 : X0) + li;
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) ss += sumsq8(__builtin_bit_cast(u32x4, qf[a][ks]));
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    if (lg == 0) cf[3][t] = t < nvalid ? (l2norm ? rsqrtf(ss + 1e-6f) : 1.f) * scale : 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[a][ks] = __builtin_bit_cast(bf16x8, mask8(__builtin_bit_cast(u32x4, qf[a][ks]), t < nvalid));
  }
  if (wv == 0) {  // gamma = cumsum(g) over the pair; beta; both zero past the sequence end (HF pads with 0)
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y0 = __shfl_up(g0, off, 64), y1 = __shfl_up(g1, off, 64);
      if (lane >= off) { g0 += y0; g1 += y1; }
    }
    const float tot0 = __shfl(g0, 63, 64);
    cf[0][lane] = g0;
    cf[0][64 + lane] = tot0 + g1;
    cf[1][lane] = b0;
    cf[1][64 + lane] = b1;
  }
  lds_barrier();

  // ---- 1. K K^T and Q K^T for the wave's row tiles X0 (chunk 0) and X1 (chunk 1), all products before any store
  //         (the fp32 L blocks replace the k tile). Per column tile Y <= X1 the k rows of Y are read once and serve:
  //         L00 (X0, Y), L11 (X1, Y >= 4) as B operands; L10 (X1, Y < 4) and P (X0 / X1, Y) as A operands of the
  //         transposed tiles (positions s down each lane's 4 rows, t across the lanes).
  bf16x8 kx[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kx[a][ks] = ldf(RA, 16 * (a ? X1 : X0) + li, 32 * ks + 8 * lg);
  f32x4 lA[4], pA[4], lB[8], pB[8];
#pragma unroll
  for (int y = 0; y < 8; ++y) {
    if (y > X1) break;
    bf16x8 ky[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) ky[ks] = ldf(RA, 16 * y + li, 32 * ks + 8 * lg);
    f32x4 a1 = zero4(), a2 = zero4();
    if (y < 4) {  // L10 (transposed)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) a1 = mfma16(ky[ks], kx[1][ks], a1);
    } else {      // L11
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) a1 = mfma16(kx[1][ks], ky[ks], a1);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) a2 = mfma16(ky[ks], qf[1][ks], a2);
    lB[y] = a1;
    pB[y] = a2;
    if (y < 4 && y <= X0) {
      f32x4 a3 = zero4(), a4 = zero4();
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        a3 = mfma16(kx[0][ks], ky[ks], a3);
        a4 = mfma16(ky[ks], qf[0][ks], a4);
      }
      lA[y] = a3;
      pA[y] = a4;
    }
  }
  lds_barrier();  // the k tile (RA) is read by every wave: now it becomes L

  // epilogues. gamma is non-increasing; tile factors relative to the tile's first row r = 16 X.
  // P B-fragments of row tiles X0 (<= 3: k steps 0-1) and X1 (k steps 0-3), kmap order, zero above the diagonal
  bf16x8 pfr0[2], pfr1[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (ks < 2) pfr0[ks] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    pfr1[ks] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
  }
  auto epilogue = [&](auto aconst) {
    constexpr int a = decltype(aconst)::value;
    constexpr int NY = a ? 8 : 4;
    const int X = a ? X1 : X0;
    const float gr = cf[0][16 * X];
    // rows t = 16 X + 4 lg + r (normal tiles) and the lane's own t = 16 X + li (transposed tiles)
    f32x4 rowL, ltr;
    const f32x4 gtr = *reinterpret_cast<const f32x4*>(&cf[0][16 * X + 4 * lg]);
    {
      const f32x4 bt4 = *reinterpret_cast<const f32x4*>(&cf[1][16 * X + 4 * lg]);
      const f32x4 rk4 = *reinterpret_cast<const f32x4*>(&cf[2][16 * X + 4 * lg]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ltr[r] = -bt4[r] * rk4[r];
        rowL[r] = ltr[r] * __expf(gtr[r] - gr);
      }
    }
    const int tl = 16 * X + li;
    const float gt = cf[0][tl];
    const float rowT_L = -cf[1][tl] * cf[2][tl] * __expf(gt - gr);
    const float rowT_P = cf[3][tl] * __expf(gt - gr);
    auto put_p = [&](int y, const float (&pv)[4]) {
      const u32x2 pk = pack4(pv[0], pv[1], pv[2], pv[3]);
      bf16x8& slot = a ? pfr1[y >> 1] : pfr0[(y >> 1) & 1];
      u32x4 cur = __builtin_bit_cast(u32x4, slot);
      if (y & 1) { cur.z = pk.x; cur.w = pk.y; } else { cur.x = pk.x; cur.y = pk.y; }
      slot = __builtin_bit_cast(bf16x8, cur);
    };
    float* Ac = Am + a * 64 * kFS;
    // one uniform branch per tile: the diagonal tile (exact per-element decay, masked) or a tile below it
#pragma unroll
    for (int y = 0; y < NY; ++y) {
      if (y > X) break;
      // normal-tile column s = 16 y + li; transposed-tile rows s = 16 y + 4 lg + r
      const int sn = 16 * y + li;
      f32x4 accP, accL;
      if constexpr (a) { accP = pB[y]; accL = lB[y]; } else { accP = pA[y]; accL = lA[y]; }
      const f32x4 gsT = *reinterpret_cast<const f32x4*>(&cf[0][16 * y + 4 * lg]);
      const f32x4 rkT = *reinterpret_cast<const f32x4*>(&cf[2][16 * y + 4 * lg]);
      if (y == X) {
        // P (transposed, s <= t) and L00 / L11 (normal, s < t)
        float pv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int sp = 16 * y + 4 * lg + r;
          pv[r] = sp <= tl ? cf[3][tl] * rkT[r] * __expf(gt - gsT[r]) * accP[r] : 0.f;
        }
        put_p(y, pv);
        const float rks = cf[2][sn], gs = cf[0][sn];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * X + 4 * lg + r;
          Ac[(t - 64 * a) * kFS + (sn - 64 * a)] = sn < t ? ltr[r] * rks * __expf(gtr[r] - gs) * accL[r] : 0.f;
        }
      } else {
        f32x4 colT;
#pragma unroll
        for (int r = 0; r < 4; ++r) colT[r] = rkT[r] * __expf(gr - gsT[r]);
        float pv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pv[r] = rowT_P * colT[r] * accP[r];
        put_p(y, pv);
        if (a == 1 && y < 4) {
          // L10 (transposed): rows s of tile y (chunk 0), column t = tl (chunk 1)
          float lv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) lv[r] = rowT_L * colT[r] * accL[r];
          *reinterpret_cast<u32x2*>(reinterpret_cast<char*>(&L10f[(X1 - 4) * 2 + (y >> 1)][lane]) + 8 * (y & 1)) =
              pack4(lv[0], lv[1], lv[2], lv[3]);
        } else {
          // L00 (X0, y) or L11 (X1, y >= 4), normal orientation: rows t = 16 X + 4 lg + r, column s = sn
          const float colN = cf[2][sn] * __expf(gr - cf[0][sn]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 16 * X + 4 * lg + r;
            Ac[(t - 64 * a) * kFS + (sn - 64 * a)] = rowL[r] * colN * accL[r];
          }
        }
      }
    }
  };
  epilogue(std::integral_constant<int, 0>{});
  epilogue(std::integral_constant<int, 1>{});
  lds_barrier();

  // ---- 2. the per-position factors of the later phases (in place, one position per thread); V loads go out; the
  //         two inverses (fp32, in place in RA)
  if (tid < kP) {
    const float gt = cf[0][tid], gl = cf[0][kP - 1], bt = cf[1][tid], rk = cf[2][tid], qs = cf[3][tid];
    cf[4][tid] = bt * __expf(gt) * rk;
    cf[2][tid] = rk * __expf(gl - gt);
    cf[3][tid] = qs * __expf(gt);
    if (tid == 0) *reinterpret_cast<float*>(rec + kRecE) = __expf(gl);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) raw[i] = raw8(vb + min(8 * ur + i, nvalid - 1) * vstride + 8 * uc);
  invert64x2(Am, wv, lane);
  lds_barrier();

  // A fragments of T00 (natural k order, columns scaled by W's or U's input factor) and of T11 (kmap order), rows
  // 16 X + li; fragments wholly above the diagonal are zero
  const bool isW = wv < 2;
  const float* cin = cf[isW ? 4 : 1];
  bf16x8 t00[4][2], t11[4][2];
#pragma unroll
  for (int X = 0; X < 4; ++X) {
    const int t = 16 * X + li;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 f0, f1;
#pragma unroll
      for (int j = 0; j < 8; ++j) { f0[j] = (__bf16)0.f; f1[j] = (__bf16)0.f; }
      if (ks <= (X >> 1)) {
        const int s0 = 32 * ks + 8 * lg;
        const f32x4 u0 = *reinterpret_cast<const f32x4*>(Am + t * kFS + s0);
        const f32x4 u1 = *reinterpret_cast<const f32x4*>(Am + t * kFS + s0 + 4);
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(cin + s0);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(cin + s0 + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int s = s0 + j;
          const float tv = j < 4 ? u0[j] : u1[j - 4];
          const float val = s < t ? tv : (s == t ? 1.f : 0.f);
          f0[j] = (__bf16)(val * (j < 4 ? c0[j] : c1[j - 4]));
        }
        const float* A1 = Am + 64 * kFS;
        const int sa = 32 * ks + 4 * lg, sb = 32 * ks + 16 + 4 * lg;
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(A1 + t * kFS + sa);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(A1 + t * kFS + sb);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int s = j < 4 ? sa + j : sb + j - 4;
          const float tv = j < 4 ? v0[j] : v1[j - 4];
          f1[j] = (__bf16)(s < t ? tv : (s == t ? 1.f : 0.f));
        }
      }
      t00[X][ks] = f0;
      t11[X][ks] = f1;
    }
  }
  lds_barrier();  // T is read: RA becomes V^T
#pragma unroll
  for (int i = 0; i < 8; ++i) raw[i] = mask8(raw[i], 8 * ur + i < nvalid);
#pragma unroll
  for (int e = 0; e < 8; ++e)
    *reinterpret_cast<u32x4*>(RA + (8 * uc + e) * kRS + 16 * (ur ^ ((uc >> 1) & 7))) = column8(raw, e);
  lds_barrier();

  // ---- 3-5. X0 = T00 diag(c) K0 (or V0), Z = L10 X0 + diag(c) K1, X1 = T11 Z, for this wave's value tiles D0 + D.
  //           The results stay in registers as 32-wide k steps over positions (kmap order).
  const int D0 = 4 * (wv & 1);
  const char* src = isW ? RB : RA;  // K^T or V^T
  bf16x8 xn[4][4];                  // [D][position k step]
  {
    bf16x8 bs[4][2];
#pragma unroll
    for (int D = 0; D < 4; ++D)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) bs[D][ks] = ldf_t(src, D0 + D, li, 32 * ks + 8 * lg);
    f32x4 x0[4][4];
#pragma unroll
    for (int X = 0; X < 4; ++X)
#pragma unroll
      for (int D = 0; D < 4; ++D) {
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          if (ks <= (X >> 1)) acc = mfma16(t00[X][ks], bs[D][ks], acc);
        x0[X][D] = acc;
      }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int D = 0; D < 4; ++D) xn[D][kt] = pack8(x0[2 * kt][D], x0[2 * kt + 1][D]);
  }
  // V^T is last read by Z: the P fragments go to LDS before X1 is formed, so that they are out of registers where
  // the most values are live
  bf16x8 zf[4][2];
  {
    f32x4 z[4][4];
#pragma unroll
    for (int X = 0; X < 4; ++X) {
      const f32x4 c = *reinterpret_cast<const f32x4*>(&cin[64 + 16 * X + 4 * lg]);
      bf16x8 la[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) la[ks] = L10f[X * 2 + ks][lane];
#pragma unroll
      for (int D = 0; D < 4; ++D) {
        const f32x4 x = unpack4(*reinterpret_cast<const u32x2*>(src + (16 * (D0 + D) + li) * kRS +
                                                              tsw(D0 + D, 64 + 16 * X + 4 * lg)));
        f32x4 acc = scale4(x, c);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) acc = mfma16(la[ks], xn[D][ks], acc);
        z[X][D] = acc;
      }
    }
#pragma unroll
    for (int D = 0; D < 4; ++D)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) zf[D][ks] = pack8(z[2 * ks][D], z[2 * ks + 1][D]);
  }
  lds_barrier();  // V^T (RA) and K^T (RB) are read: RA takes the P fragments, RB becomes K~^T in place
  {
    bf16x8* Pf = reinterpret_cast<bf16x8*>(RA);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks < 2 && ks <= (X0 >> 1)) Pf[(pbase(X0) + ks) * 64 + lane] = pfr0[ks];
      if (ks <= (X1 >> 1)) Pf[(pbase(X1) + ks) * 64 + lane] = pfr1[ks];
    }
    // K~[t][d] = k[t][d] rk_t e^(gamma_last - gamma_t): chunk j of row d holds positions 8 (j ^ (d / 16 % 8)) .. + 7
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = tid + 256 * i, d = c >> 4, j = c & 15;
      u32x4* p = reinterpret_cast<u32x4*>(RB + d * kRS + 16 * j);
      const int t0s = 8 * (j ^ ((d >> 4) & 7));
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(&cf[2][t0s]);
      const f32x4 s1 = *reinterpret_cast<const f32x4*>(&cf[2][t0s + 4]);
      const u32x4 w = *p;
      const f32x4 a = unpack4(u32x2{w.x, w.y}), bb = unpack4(u32x2{w.z, w.w});
      const u32x2 lo = pack4(a[0] * s0[0], a[1] * s0[1], a[2] * s0[2], a[3] * s0[3]);
      const u32x2 hi = pack4(bb[0] * s1[0], bb[1] * s1[1], bb[2] * s1[2], bb[3] * s1[3]);
      *p = u32x4{lo.x, lo.y, hi.x, hi.y};
    }
  }
  {
    f32x4 x1[4][4];
#pragma unroll
    for (int X = 0; X < 4; ++X)
#pragma unroll
      for (int D = 0; D < 4; ++D) {
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          if (ks <= (X >> 1)) acc = mfma16(t11[X][ks], zf[D][ks], acc);
        x1[X][D] = acc;
      }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int D = 0; D < 4; ++D) xn[D][2 + kt] = pack8(x1[2 * kt][D], x1[2 * kt + 1][D]);
  }
  lds_barrier();  // the P fragments and K~^T are in LDS

  // q values of the Q' products (W waves: rows t = 16 X + li, columns 16 (D0 + D) + 4 lg ..), loaded ahead of use:
  // row tiles 0-1 before the M products, 2-7 after them
  u32x2 qpre[8][4];
  auto load_q = [&](int X) {
    const __bf16* qr = qb + min(16 * X + li, nvalid - 1) * kstride;
#pragma unroll
    for (int D = 0; D < 4; ++D) qpre[X][D] = *reinterpret_cast<const u32x2*>(qr + 16 * (D0 + D) + 4 * lg);
  };
  if (isW) {
#pragma unroll
    for (int X = 0; X < 1; ++X) load_q(X);
  }

  // ---- 6. W waves: M^T = -W^T K~ (rows d' = 16 (D0 + D) .., columns d = 16 E ..), stored as M's A fragments;
  //         U waves: Bm = K~^T U (rows d = 16 E .., columns dv = 16 (D0 + D) ..), stored in D order.
#pragma unroll
  for (int E = 0; E < 8; ++E) {
    bf16x8 kf[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) kf[kt] = ldf_km_t(RB, E, li, 32 * kt, lg);
    if (isW) {
      f32x4 acc[4];
#pragma unroll
      for (int D = 0; D < 4; ++D) {
        acc[D] = zero4();
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) acc[D] = mfma16(xn[D][kt], kf[kt], acc[D]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[D][r] = -acc[D][r];
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        *reinterpret_cast<bf16x8*>(rec + kRecM + ((size_t)(E * 4 + (D0 >> 1) + hh) * 64 + lane) * 16) =
            pack8(acc[2 * hh], acc[2 * hh + 1]);
    } else {
#pragma unroll
      for (int D = 0; D < 4; ++D) {
        f32x4 acc = zero4();
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) acc = mfma16(kf[kt], xn[D][kt], acc);
        *reinterpret_cast<u32x2*>(rec + kRecB + ((size_t)(E * 8 + D0 + D) * 64 + lane) * 8) =
            pack4(acc[0], acc[1], acc[2], acc[3]);
      }
    }
  }

  // ---- 7. W waves: Q'^T = Q^ e^gamma - W^T P^T (rows d', columns t), stored as Q''s A fragments; U waves:
  //         R^T = U^T P^T (rows dv, columns t), stored in transposed D order. P is zero above the diagonal: row tile X
  //         has X / 2 + 1 k steps.
  const bf16x8* Pf = reinterpret_cast<const bf16x8*>(RA);
  if (isW) {
#pragma unroll
    for (int X = 1; X < 8; ++X) load_q(X);
  }
#pragma unroll
  for (int X = 0; X < 8; ++X) {
    const int t = 16 * X + li;
    bf16x8 pf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) pf[ks] = Pf[(pbase(X) + min(ks, X >> 1)) * 64 + lane];
    if (isW) {
      const float cq = cf[3][t];
      f32x4 acc[4];
#pragma unroll
      for (int D = 0; D < 4; ++D) {
        const f32x4 qv = unpack4(qpre[X][D]);
        f32x4 pw = zero4();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          if (ks <= (X >> 1)) pw = mfma16(xn[D][ks], pf[ks], pw);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[D][r] = qv[r] * cq - pw[r];
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        *reinterpret_cast<bf16x8*>(rec + kRecQ + ((size_t)(X * 4 + (D0 >> 1) + hh) * 64 + lane) * 16) =
            pack8(acc[2 * hh], acc[2 * hh + 1]);
    } else {
#pragma unroll
      for (int D = 0; D < 4; ++D) {
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          if (ks <= (X >> 1)) acc = mfma16(xn[D][ks], pf[ks], acc);
        *reinterpret_cast<u32x2*>(rec + kRecR + ((size_t)(X * 8 + D0 + D) * 64 + lane) * 8) =
            pack4(acc[0], acc[1], acc[2], acc[3]);
      }
    }
  }
}

// Blocks are dispatched round-robin over the 8 XCDs (block i runs on XCD i % 8). The 16 blocks of one (row, head)
// read the same records, so they are mapped onto one XCD to share its L2: block L serves XCD x = L % 8, and the j-th
// block of that XCD (j = L / 8) is block j % 16 of unit 8 (j / 16) + x. When the number of (row, head) units is not
// a multiple of 8 the plain mapping is used.
__device__ __forceinline__ void scan_coords(int L, int nunits, int& idx, int& unit) {
  if ((nunits & 7) == 0) {
    const int x = L & 7, j = L >> 3;
    idx = j & 15;
    unit = 8 * (j >> 4) + x;
  } else {
    idx = L & 15;
    unit = L >> 4;
  }
}


// Operands of one pair for one wave of the scan kernel: a state-row-tile wave takes the M fragments and the Bm piece
// of its tile, an output-tile wave the Q' fragments and the R piece of its tile.
struct StateOps {
  bf16x8 m[4];
  u32x2 bv;
  float eg;
};
struct OutOps {
  bf16x8 qf[4];
  u32x2 rv;
};

constexpr int kScanThreads = 12 * 64;

// The pair loop of a scan wave with its operands kScanAhead pairs ahead: slot i of `ops` serves the pairs i mod
// kScanAhead. Whole groups of kScanAhead pairs run without conditions and in program order (the scheduling barriers
// keep each pair's loads behind its step, so that the wait counts allow the full prefetch distance), then the rest.
template <typename Ops, typename Load, typename Step>
__device__ __forceinline__ void pipeline(int NP, Ops (&ops)[kScanAhead], Load load, Step step) {
#pragma unroll
  for (int i = 0; i < kScanAhead; ++i) {
    load(i, ops[i]);
    __builtin_amdgcn_sched_barrier(0);
  }
  int pp = 0;
  for (; pp + kScanAhead <= NP; pp += kScanAhead) {
#pragma unroll
    for (int i = 0; i < kScanAhead; ++i) {
      step(pp + i, ops[i]);
      load(pp + i + kScanAhead, ops[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int i = 0; i + 1 < kScanAhead; ++i)
    if (pp + i < NP) step(pp + i, ops[i]);
}

// Waves 0-7: state row tile w (rows 16 w .. 16 w + 15 of the block's 128 x 16 slice), S <- e^G S + Bm + M S.
// Waves 8-11: output row tile 4 half + (w - 8) of the pair, O = Q' S + R.
// Each state wave publishes its tile as bf16 once per pair (LDS, double-buffered by pair parity); after the pair's
// barrier every wave reads the whole bf16 slice as its B operands. A wave holds the operands of three pairs ahead.
__global__ __launch_bounds__(kScanThreads, 1) void gdn_pair_scan_kernel(const char* __restrict__ ws, const float* s_in,
                                                                        float* s_out, __bf16* __restrict__ o, int T,
                                                                        int NP, int H, int B) {
  __shared__ u32x2 slot[2][8][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int idx, unit;
  scan_coords(blockIdx.x, H * B, idx, unit);
  const int sl = idx & 7, half = idx >> 3;
  const int h = unit % H, b = unit / H;
  const int li = lane & 15, lg = lane >> 4;
  const char* rec0 = ws + (size_t)unit * NP * kRecBytes;
  const int col = 16 * sl + li;

  // Outputs go through a buffer resource spanning row b's [T, H, 128] block: stores past the sequence end fall
  // outside it and are dropped by the hardware. Lane (li, lg) of output tile ot holds value columns
  // 16 sl + 4 lg .. + 3 of position 16 ot + li (byte offset below).
  const __amdgpu_buffer_rsrc_t orc = __builtin_amdgcn_make_buffer_rsrc(
      o + (size_t)b * T * H * kD, 0, (int)((size_t)T * H * kD * sizeof(__bf16)), 0x00020000);
  auto out_off = [&](int pp, int ot) { return ((kP * pp + 16 * ot + li) * H + h) * kD * 2 + (16 * sl + 4 * lg) * 2; };

  auto gather = [&](int pp, bf16x8 (&sb)[4]) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x2 lo = slot[pp & 1][2 * ks][lane], hi = slot[pp & 1][2 * ks + 1][lane];
      const u32x4 v = {lo.x, lo.y, hi.x, hi.y};
      sb[ks] = __builtin_bit_cast(bf16x8, v);
    }
  };

  if (w < 8) {
    // ---------------- state row tile w ----------------
    const size_t sbase = (size_t)unit * kD * kD;
    f32x4 S;
#pragma unroll
    for (int r = 0; r < 4; ++r) S[r] = s_in ? s_in[sbase + (size_t)(16 * w + 4 * lg + r) * kD + col] : 0.f;
    auto load = [&](int pp, StateOps& op) {
      const char* rec = rec0 + (size_t)min(pp, NP - 1) * kRecBytes;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        op.m[ks] = *reinterpret_cast<const bf16x8*>(rec + kRecM + ((size_t)(w * 4 + ks) * 64 + lane) * 16);
      op.bv = *reinterpret_cast<const u32x2*>(rec + kRecB + ((size_t)(w * 8 + sl) * 64 + lane) * 8);
      op.eg = *reinterpret_cast<const float*>(rec + kRecE);
    };
    auto step = [&](int pp, const StateOps& op) {
      slot[pp & 1][w][lane] = pack4(S[0], S[1], S[2], S[3]);
      lds_barrier();
      bf16x8 sb[4];
      gather(pp, sb);
      const f32x4 bm = unpack4(op.bv);
      f32x4 s;
#pragma unroll
      for (int r = 0; r < 4; ++r) s[r] = op.eg * S[r] + bm[r];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) s = mfma16(op.m[ks], sb[ks], s);
      S = s;
    };
    StateOps ops[kScanAhead];
    pipeline(NP, ops, load, step);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (s_out && half == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s_out[sbase + (size_t)(16 * w + 4 * lg + r) * kD + col] = S[r];
    }
    return;
  }

  // ---------------- output row tile 4 half + j ----------------
  const int ot = 4 * half + (w - 8);
  auto load = [&](int pp, OutOps& op) {
    const char* rec = rec0 + (size_t)min(pp, NP - 1) * kRecBytes;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      op.qf[ks] = *reinterpret_cast<const bf16x8*>(rec + kRecQ + ((size_t)(ot * 4 + ks) * 64 + lane) * 16);
    op.rv = *reinterpret_cast<const u32x2*>(rec + kRecR + ((size_t)(ot * 8 + sl) * 64 + lane) * 8);
  };
  // O^T = S^T Q'^T + R^T: the state fragments as the A operand and Q' as B, so that lane (li, lg) holds value
  // columns 16 sl + 4 lg .. + 3 of position 16 ot + li (8 bytes).
  auto step = [&](int pp, const OutOps& op) {
    lds_barrier();
    bf16x8 sb[4];
    gather(pp, sb);
    f32x4 acc = unpack4(op.rv);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = mfma16(sb[ks], op.qf[ks], acc);
    __builtin_amdgcn_raw_buffer_store_b64(pack4(acc[0], acc[1], acc[2], acc[3]), orc, out_off(pp, ot), 0, 0);
  };
  OutOps ops[kScanAhead];
  pipeline(NP, ops, load, step);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ================================================================================================================
// fp32 path (fp32 q, k, v): the chunk-64 WY form of HF:281-327 with every product in fp32
// (v_mfma_f32_16x16x4_f32), so that outputs and state agree with the fp32 recurrence to fp32 rounding.
//
// Kernel F1, gdn_f32_prep_kernel: one 256-thread block per (chunk, head, row), all chunks in parallel. With
// k^ = l2norm(k), q^ = l2norm(q) * scale and gamma = cumsum(g) inside the chunk it writes one record of
//   W   [64 pos][128 d]  = T diag(beta e^gamma) K^          U  [64 pos][128 dv] = T diag(beta) V
//   Qe  [64 pos][128 d]  = Q^ e^gamma (0 past the end)      Kt [128 d][64 pos]  = (K^ e^(gamma_last - gamma))^T
//   P   [64 t][64 s]     = (q^_t . k^_s) e^(gamma_t - gamma_s) for s <= t (lower triangle only)
//   e^gamma_last,  with T = (I - L)^-1, L[t][s] = -beta_t (k^_t . k^_s) e^(gamma_t - gamma_s) (s < t).
// Kernel F2, gdn_f32_scan_kernel: 8 blocks per (row, head), one per 16 value columns (4 blocks of 32 columns when 8
// per (row, head) would exceed the 256 blocks that are resident at once); each carries its 128 x 16 (or 32) fp32
// state slice in registers (wave w: state rows 32 w .. 32 w + 31) and per chunk computes
//   V = U - W S,   O = Qe S + P V,   S <- e^gamma_last S + Kt V
// (wave w: positions 16 w .. 16 w + 15 of V and O). The state and V tiles are exchanged through LDS.
//
// Product layout: an operand X[m][k] held row-major feeds the A (or B) side of a 16 x 16 x 4 MFMA group over one
// 16-wide k chunk as one float4 per lane (X[m][16 c + 4 g .. + 3], m = lane % 16, g = lane / 16), step s using
// element s, i.e. k index 16 c + 4 g + s. A 16 x 16 accumulator tile in D layout (lane: column lane % 16, rows
// 4 g + r in element r) supplies the other side of the same four steps directly: element s of lane l is row
// 4 g + s. The k permutation is the same on both sides, so the sum is unchanged.
constexpr int kFX = 132;                 // row stride (floats) of the fp32 [64][128] staging tiles
constexpr size_t kFRecW = 0;             // W   [64][128]
constexpr size_t kFRecU = 32768;         // U   [64][128]
constexpr size_t kFRecQ = 65536;         // Qe  [64][128]
constexpr size_t kFRecK = 98304;         // Kt  [128][64]
constexpr size_t kFRecP = 131072;        // P   [64][64]
constexpr size_t kFRecE = 147456;        // e^gamma_last
constexpr size_t kFRecBytes = 147712;    // 256-byte aligned

// acc += X Y over one 16-wide k chunk (layouts above): x = X[m][16 c + 4 g ..], y = element s at k = 16 c + 4 g + s
__device__ __forceinline__ f32x4 mm_k16(const f32x4& x, const f32x4& y, f32x4 acc) {
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma_f32_16x16x4(x[s], y[s], acc);
  return acc;
}

// Front-end form (the Gated DeltaNet layer's conv + SiLU and gate terms run in the prep kernel's load phase, so q, k,
// v, g and beta never reach HBM): the fused projection output y [B, T, ldy] with the q | k | v channels (C = 2 Kd +
// Vd, K = 4 taps, weights [C][4], optional bias [C]) from column 0 and the b, a columns of head h at b_off + h,
// a_off + h; the carried conv state [B, 3, C] holds the 3 inputs before y's first token. Only the first chunk's prep
// blocks read the state; the scan kernel, which starts after every prep block has ended, advances it to the last 3
// inputs of [old state | y]: no block reads a state entry that another block of the same launch writes.
constexpr int kFrontK = 4;
struct GdnFront {
  const float* y;
  int64_t ldy;
  const float* cw;      // [C][kFrontK]
  const float* cb;      // [C] or null
  float* cst;           // [B][kFrontK - 1][C]
  const float* A_log;   // [H]
  const float* dt_bias; // [H]
  int b_off, a_off, C, Kd;
};

template <bool FE>
__global__ __launch_bounds__(256, 1) void gdn_f32_prep_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                              const float* __restrict__ v, const float* __restrict__ g,
                                                              const float* __restrict__ beta, char* __restrict__ ws,
                                                              int T, int NC, int Hk, int H, float scale, int l2norm,
                                                              GdnFront fe) {
  __shared__ __attribute__((aligned(16))) float Ks[kC * kFX];   // k rows (unnormalised)
  __shared__ __attribute__((aligned(16))) float Xs[kC * kFX];   // q rows, then v rows
  __shared__ __attribute__((aligned(16))) float Am[kC * kFS];   // L -> T (invert64 layout) -> T dense
  __shared__ float scr[4][16 * 17];
  __shared__ float gam[kC], bet[kC], rkn[kC], rqn[kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int kh = h / (H / Hk);
  const int t0 = c * kC;
  const int nvalid = min(kC, T - t0);
  char* rec = ws + (((size_t)b * H + h) * NC + c) * kFRecBytes;
  float* recf = reinterpret_cast<float*>(rec);

  // ---- stage k and q (thread: row tid / 4, columns 32 (tid % 4) .. + 31), the gates, the l2 norms
  const int row = tid >> 2, c0 = (tid & 3) * 32;
  const bool valid = row < nvalid;
  const size_t tok = (size_t)b * T + t0 + min(row, nvalid - 1);
  f32x4 kr[8];  // the thread's k row; then v, held until q is no longer needed
  float g0 = 0.f, b0 = 0.f;
  auto norms = [&](const f32x4(&kk)[8], const f32x4(&qq)[8]) {  // l2 norms of the thread's row (4 threads a row)
    float ssk = 0.f, ssq = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) { ssk += kk[j][e] * kk[j][e]; ssq += qq[j][e] * qq[j][e]; }
    ssk += __shfl_xor(ssk, 1, 64);
    ssk += __shfl_xor(ssk, 2, 64);
    ssq += __shfl_xor(ssq, 1, 64);
    ssq += __shfl_xor(ssq, 2, 64);
    if ((tid & 3) == 0) {
      rkn[row] = l2norm ? rsqrtf(ssk + 1e-6f) : 1.f;
      rqn[row] = l2norm ? rsqrtf(ssq + 1e-6f) : 1.f;
    }
  };
  if constexpr (FE) {
    // causal conv + SiLU of the head's k, q and v channels of y (thread: channel quad cq, tokens 8 tg .. 8 tg + 7 of
    // the chunk; the 3 inputs before the chunk from y, or for the first chunk from the carried state), zero past the
    // sequence end; the gate terms from the b and a columns. The front-end kernel's arithmetic in its order; the
    // norms are then taken over the staged rows in the order of the other form.
    const int cq = tid & 31, tg = tid >> 5;
    constexpr int kWin = 8 + kFrontK - 1;  // inputs of tokens t0 + 8 tg - 3 .. t0 + 8 tg + 7
    // every load of the three windows is issued before any is used: one memory round trip. Offsets are 32-bit
    // relative to the row's first token of the chunk (the launcher bounds ldy) and to the row's conv state.
    const float* ybase = fe.y + ((size_t)b * T + t0) * fe.ldy;
    const float* sbase = fe.cst + (size_t)b * (kFrontK - 1) * fe.C;
    auto window = [&](int ch, f32x4(&win)[kWin]) {
#pragma unroll
      for (int j = 0; j < kWin; ++j) {
        const int r = t0 + 8 * tg + j - (kFrontK - 1);
        const float* py = ybase + ((min(r, T - 1) - t0) * (int)fe.ldy + ch);
        const float* ps = sbase + ((kFrontK - 1 + min(r, -1)) * fe.C + ch);
        win[j] = *reinterpret_cast<const f32x4*>(r >= 0 ? py : ps);
      }
    };
    auto taps = [&](int ch, f32x4(&tw)[4], f32x4& bias) {  // tw[e][i]: tap i of channel ch + e
      const f32x4* cw4 = reinterpret_cast<const f32x4*>(fe.cw + (size_t)ch * kFrontK);
#pragma unroll
      for (int e = 0; e < 4; ++e) tw[e] = cw4[e];
      bias = fe.cb ? *reinterpret_cast<const f32x4*>(fe.cb + ch) : zero4();
    };
    auto conv = [&](const f32x4(&win)[kWin], const f32x4(&tw)[4], const f32x4& bias, f32x4(&res)[8]) {
#pragma unroll
      for (int o = 0; o < 8; ++o) {
        f32x4 acc = bias;
#pragma unroll
        for (int i = 0; i < kFrontK; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[e] += tw[e][i] * win[o + i][e];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = silu_f(acc[e]);
        res[o] = 8 * tg + o < nvalid ? acc : zero4();
      }
    };
    const int chk = fe.Kd + kh * kD + 4 * cq, chq = kh * kD + 4 * cq, chv = 2 * fe.Kd + h * kD + 4 * cq;
    f32x4 wk[kWin], wq[kWin], wv[kWin], tk[4], tq[4], tv[4], bk, bq, bv;
    window(chk, wk);
    taps(chk, tk, bk);
    window(chq, wq);
    taps(chq, tq, bq);
    window(chv, wv);
    taps(chv, tv, bv);
    // the gate inputs of the chunk's tokens (lane = token; used by wave 0, loaded by every wave), issued with the
    // windows
    const float* yr = ybase + min(lane, nvalid - 1) * (int)fe.ldy;
    const float gin_b = yr[fe.b_off + h], gin_a = yr[fe.a_off + h], gin_A = fe.A_log[h], gin_dt = fe.dt_bias[h];
    f32x4 cr[8];
    conv(wk, tk, bk, cr);
#pragma unroll
    for (int o = 0; o < 8; ++o) *reinterpret_cast<f32x4*>(Ks + (8 * tg + o) * kFX + 4 * cq) = cr[o];
    conv(wq, tq, bq, cr);
#pragma unroll
    for (int o = 0; o < 8; ++o) *reinterpret_cast<f32x4*>(Xs + (8 * tg + o) * kFX + 4 * cq) = cr[o];
    conv(wv, tv, bv, kr);
    // the gate inputs are consumed here, so that the compiler keeps their loads with the windows rather than
    // sinking them into the branch below (a second memory round trip for wave 0)
    asm volatile("" ::"v"(gin_b), "v"(gin_a));
    if (wave == 0 && lane < nvalid) {
      b0 = sigmoidf_(gin_b);
      g0 = -__expf(gin_A) * softplus_f(gin_a + gin_dt);
    }
    __syncthreads();
    f32x4 ka[8], qa[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ka[j] = *reinterpret_cast<const f32x4*>(Ks + row * kFX + c0 + 4 * j);
      qa[j] = *reinterpret_cast<const f32x4*>(Xs + row * kFX + c0 + 4 * j);
    }
    norms(ka, qa);
  } else {
    f32x4 xr[8];
    const float* kp = k + (tok * Hk + kh) * kD + c0;
    const float* qp = q + (tok * Hk + kh) * kD + c0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      kr[j] = *reinterpret_cast<const f32x4*>(kp + 4 * j);
      xr[j] = *reinterpret_cast<const f32x4*>(qp + 4 * j);
    }
    if (wave == 0 && lane < nvalid) {
      const size_t gi = ((size_t)b * T + t0 + lane) * H + h;
      g0 = g[gi];
      b0 = beta[gi];
    }
    norms(kr, xr);
    const f32x4 z = zero4();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      *reinterpret_cast<f32x4*>(Ks + row * kFX + c0 + 4 * j) = valid ? kr[j] : z;
      *reinterpret_cast<f32x4*>(Xs + row * kFX + c0 + 4 * j) = valid ? xr[j] : z;
    }
  }
  if (wave == 0) {  // gamma = cumsum(g) over the chunk; g = beta = 0 past the sequence end (HF pads with zeros)
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(g0, off, 64);
      if (lane >= off) g0 += y;
    }
    gam[lane] = g0;
    bet[lane] = b0;
  }
  if constexpr (!FE) {  // v rows, loaded now and staged once q is no longer needed
    const float* vp = v + (tok * H + h) * kD + c0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(vp + 4 * j);
      kr[j] = valid ? t : zero4();  // kr is free: k is in LDS
    }
  }
  __syncthreads();

  // ---- K K^T -> L (strictly lower, into Am) and Q K^T -> P (lower triangle incl. the diagonal, to the record). Wave
  //      w takes the L row tile w (w + 1 tiles) and the P row tile 3 - w (4 - w tiles).
  {
    auto tile = [&](const float* X, int i, int j) {
      f32x4 acc = zero4();
#pragma unroll
      for (int kc = 0; kc < 8; ++kc) {
        const f32x4 xa = *reinterpret_cast<const f32x4*>(X + (16 * i + li) * kFX + 16 * kc + 4 * lg);
        const f32x4 yb = *reinterpret_cast<const f32x4*>(Ks + (16 * j + li) * kFX + 16 * kc + 4 * lg);
        acc = mm_k16(xa, yb, acc);
      }
      return acc;
    };
    const int iL = wv, iP = 3 - wv;
    for (int j = 0; j <= iL; ++j) {
      const f32x4 acc = tile(Ks, iL, j);
      const int s = 16 * j + li;
      const float ps = rkn[s], gs = gam[s];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * iL + 4 * lg + r;
        Am[t * kFS + s] = s < t ? -bet[t] * rkn[t] * ps * acc[r] * __expf(gam[t] - gs) : 0.f;
      }
    }
    for (int j = 0; j <= iP; ++j) {
      const f32x4 acc = tile(Xs, iP, j);
      const int s = 16 * j + li;
      const float ps = rkn[s], gs = gam[s];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * iP + 4 * lg + r;
        recf[kFRecP / 4 + t * kC + s] = s <= t ? rqn[t] * scale * ps * acc[r] * __expf(gam[t] - gs) : 0.f;
      }
    }
  }
  // ---- Qe = Q^ e^gamma (thread: its staged row and columns)
  {
    const float f = valid ? rqn[row] * scale * __expf(gam[row]) : 0.f;
    float* dst = recf + kFRecQ / 4 + row * kD + c0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(Xs + row * kFX + c0 + 4 * j);
      f32x4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = x[e] * f;
      *reinterpret_cast<f32x4*>(dst + 4 * j) = y;
    }
  }
  __syncthreads();

  // ---- T = (I - L)^-1, then dense (zeros above the diagonal) in place; v replaces q in Xs
  invert64(Am, wv, lane, scr[wave], [] { __syncthreads(); });
  __syncthreads();
  {
    float tv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int idx = tid + 256 * e;
      tv[e] = tinv(Am, idx >> 6, idx & 63);
    }
    // v: the thread's row (or in the front-end form its channel quad and tokens)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float* dst = FE ? Xs + (8 * (tid >> 5) + j) * kFX + 4 * (tid & 31) : Xs + row * kFX + c0 + 4 * j;
      *reinterpret_cast<f32x4*>(dst) = kr[j];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int idx = tid + 256 * e;
      Am[(idx >> 6) * kFS + (idx & 63)] = tv[e];
    }
  }
  __syncthreads();

  // ---- W = T diag(beta e^gamma rk) K, U = T diag(beta) V. Wave w: column tiles 2 w, 2 w + 1 of both, all four row
  //      tiles (T is lower triangular: row tile i sums k chunks 0..i).
  {
    f32x4 ta[4][4];  // T[16 i + li][16 kc + 4 lg ..]
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int kc = 0; kc < 4; ++kc)
        ta[i][kc] = kc <= i ? *reinterpret_cast<const f32x4*>(Am + (16 * i + li) * kFS + 16 * kc + 4 * lg) : zero4();
#pragma unroll
    for (int m = 0; m < 2; ++m) {  // 0: W from k, 1: U from v
      const float* src = m == 0 ? Ks : Xs;
      float* dst = recf + (m == 0 ? kFRecW : kFRecU) / 4;
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int d = 16 * (2 * wv + a) + li;
        f32x4 yb[4];  // scaled operand rows s = 16 kc + 4 lg + e at column d
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int s = 16 * kc + 4 * lg + e;
            const float f = m == 0 ? bet[s] * __expf(gam[s]) * rkn[s] : bet[s];
            yb[kc][e] = src[s * kFX + d] * f;
          }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 acc = zero4();
#pragma unroll
          for (int kc = 0; kc <= i; ++kc) acc = mm_k16(ta[i][kc], yb[kc], acc);
#pragma unroll
          for (int r = 0; r < 4; ++r) dst[(16 * i + 4 * lg + r) * kD + d] = acc[r];
        }
      }
    }
  }
  // ---- Kt = (K^ e^(gamma_last - gamma))^T: thread writes Kt[d][s] for s = tid % 64, d = tid / 64 + 4 e
  {
    const int s = tid & 63;
    const float f = rkn[s] * __expf(gam[kC - 1] - gam[s]);
    float* dst = recf + kFRecK / 4;
#pragma unroll 8
    for (int e = 0; e < 32; ++e) {
      const int d = (tid >> 6) + 4 * e;
      dst[d * kC + s] = Ks[s * kFX + d] * f;
    }
  }
  if (tid == 0) recf[kFRecE / 4] = __expf(gam[kC - 1]);
}

// Operands of one chunk for one wave of the fp32 scan (CT column tiles of 16 per block).
template <int CT>
struct F32Ops {
  f32x4 w[8];      // W rows 16 w + li, k chunks 0..7
  f32x4 qe[8];     // Qe rows 16 w + li
  f32x4 p[4];      // P row 16 w + li, position chunks 0..3 (chunks past w unused)
  f32x4 kt[2][4];  // Kt rows 32 w + 16 i + li, position chunks 0..3
  float u[CT][4];  // U rows 16 w + 4 lg + r, the block's columns
  float eg;
};

// CT column tiles of 16 per block: 8 / CT blocks per (row, head). The launcher takes CT = 2 when 8 blocks per (row,
// head) would not all be resident at once (one block per CU: 316 VGPRs); the W, Qe, P, Kt operands are then loaded
// once for two column tiles.
template <int CT>
__global__ __launch_bounds__(256, 1) void gdn_f32_scan_kernel(const char* __restrict__ ws, const float* s_in,
                                                              float* s_out, float* __restrict__ o, int T, int NC,
                                                              int H, int B, int Hk, GdnFront fe) {
  constexpr int NSL = 8 / CT;      // blocks (slices) per (row, head)
  __shared__ f32x4 sS[8][CT][64];  // state row tiles (D layout) of the four waves
  __shared__ f32x4 sV[4][CT][64];  // V row tiles
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int li = lane & 15, lg = lane >> 4;
  // the blocks of one (row, head) read the same records: place them on one XCD (block i runs on XCD i % 8)
  const int nunits = H * B, L = blockIdx.x;
  int sl, unit;
  if ((nunits & 7) == 0) {
    sl = (L >> 3) % NSL;
    unit = 8 * (L / (8 * NSL)) + (L & 7);
  } else {
    sl = L % NSL;
    unit = L / NSL;
  }
  const int h = unit % H, b = unit / H;
  int col[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) col[ct] = 16 * (CT * sl + ct) + li;
  const char* rec0 = ws + (size_t)unit * NC * kFRecBytes;
  const size_t sbase = (size_t)unit * kD * kD;

  f32x4 S[CT][2];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        S[ct][i][r] = s_in ? s_in[sbase + (size_t)(32 * w + 16 * i + 4 * lg + r) * kD + col[ct]] : 0.f;

  auto load = [&](int c, F32Ops<CT>& op) {
    const char* rec = rec0 + (size_t)min(c, NC - 1) * kFRecBytes;
    const float* rf = reinterpret_cast<const float*>(rec);
#pragma unroll
    for (int kc = 0; kc < 8; ++kc) {
      op.w[kc] = *reinterpret_cast<const f32x4*>(rf + kFRecW / 4 + (16 * w + li) * kD + 16 * kc + 4 * lg);
      op.qe[kc] = *reinterpret_cast<const f32x4*>(rf + kFRecQ / 4 + (16 * w + li) * kD + 16 * kc + 4 * lg);
    }
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
      op.p[kc] = *reinterpret_cast<const f32x4*>(rf + kFRecP / 4 + (16 * w + li) * kC + 16 * kc + 4 * lg);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int kc = 0; kc < 4; ++kc)
        op.kt[i][kc] = *reinterpret_cast<const f32x4*>(rf + kFRecK / 4 + (32 * w + 16 * i + li) * kC + 16 * kc + 4 * lg);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) op.u[ct][r] = rf[kFRecU / 4 + (16 * w + 4 * lg + r) * kD + col[ct]];
    op.eg = rf[kFRecE / 4];
  };

  auto step = [&](int c, const F32Ops<CT>& op) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      sS[2 * w][ct][lane] = S[ct][0];
      sS[2 * w + 1][ct][lane] = S[ct][1];
    }
    lds_barrier();
    f32x4 ws_[CT], oacc[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      ws_[ct] = zero4();
      oacc[ct] = zero4();
    }
#pragma unroll
    for (int kc = 0; kc < 8; ++kc)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const f32x4 sb = (kc >> 1) == w ? S[ct][kc & 1] : sS[kc][ct][lane];
        ws_[ct] = mm_k16(op.w[kc], sb, ws_[ct]);
        oacc[ct] = mm_k16(op.qe[kc], sb, oacc[ct]);
      }
    f32x4 vn[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
      for (int r = 0; r < 4; ++r) vn[ct][r] = op.u[ct][r] - ws_[ct][r];
      sV[w][ct][lane] = vn[ct];
    }
    lds_barrier();
    f32x4 Vb[CT][4];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) Vb[ct][kc] = kc == w ? vn[ct] : sV[kc][ct][lane];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        if (kc <= w) oacc[ct] = mm_k16(op.p[kc], Vb[ct][kc], oacc[ct]);
    const int tb = kC * c + 16 * w + 4 * lg;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (tb + r < T) o[(((size_t)b * T + tb + r) * H + h) * kD + col[ct]] = oacc[ct][r];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      f32x4 sn[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) sn[ct][r] = op.eg * S[ct][i][r];
#pragma unroll
      for (int kc = 0; kc < 4; ++kc)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) sn[ct] = mm_k16(op.kt[i][kc], Vb[ct][kc], sn[ct]);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) S[ct][i] = sn[ct];
    }
  };

  // front-end form: the carried conv state of this block's channels (16 CT of the head's v channels, and for the first
  // head of a k group 16 CT of its q and k channels) <- the last 3 inputs of [old state | y]; one lane per channel
  // reads its sources before writing, and no other block touches the channel
  constexpr int FCH = 16 * CT;
  const int fm = (int)threadIdx.x / FCH;
  const bool fstate = fe.cst && (int)threadIdx.x < 3 * FCH && (fm == 2 || h % (H / Hk) == 0);
  int fch = 0;
  float fnv[kFrontK - 1];
  if (fstate) {
    const int kh = h / (H / Hk);
    fch = (fm == 0 ? kh * kD : fm == 1 ? fe.Kd + kh * kD : 2 * fe.Kd + h * kD) + FCH * sl + ((int)threadIdx.x % FCH);
#pragma unroll
    for (int j = 0; j < kFrontK - 1; ++j) {
      const int src = T + j;  // index into [old state (3) | inputs (T)]
      fnv[j] = src >= kFrontK - 1 ? fe.y[((size_t)b * T + src - (kFrontK - 1)) * fe.ldy + fch]
                                  : fe.cst[((size_t)b * (kFrontK - 1) + src) * fe.C + fch];
    }
  }

  F32Ops<CT> o0, o1;
  load(0, o0);
  if (fstate) {
#pragma unroll
    for (int j = 0; j < kFrontK - 1; ++j) fe.cst[((size_t)b * (kFrontK - 1) + j) * fe.C + fch] = fnv[j];
  }
  for (int c = 0; c < NC; c += 2) {
    load(c + 1, o1);
    step(c, o0);
    if (c + 1 < NC) {
      load(c + 2, o0);
      step(c + 1, o1);
    }
  }
  if (s_out) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          s_out[sbase + (size_t)(32 * w + 16 * i + 4 * lg + r) * kD + col[ct]] = S[ct][i][r];
  }
}

// fp32 scan launch: 8 blocks per (row, head) while they fit one per CU (256 CUs), else 4 of two column tiles each
static void gdn_f32_scan_launch(const char* ws, const float* s_in, float* s_out, float* o, int T, int NC, int H,
                                int B, int Hk, const GdnFront& fe, hipStream_t st) {
  if (8 * H * B <= 256)
    hipLaunchKernelGGL(gdn_f32_scan_kernel<1>, dim3((unsigned)(8 * H * B)), dim3(256), 0, st, ws, s_in, s_out, o, T,
                       NC, H, B, Hk, fe);
  else
    hipLaunchKernelGGL(gdn_f32_scan_kernel<2>, dim3((unsigned)(4 * H * B)), dim3(256), 0, st, ws, s_in, s_out, o, T,
                       NC, H, B, Hk, fe);
}

}  // namespace q35

extern "C" size_t q35_gdn_chunk_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t Dk, int64_t Dv,
                                                int64_t chunk_size, int dtype) {
  using namespace q35;
  if (B <= 0 || T <= 0 || H <= 0 || Dk != kD || Dv != kD || chunk_size != kC) return 0;
  if (dtype == Q35_F32) return (size_t)B * H * (size_t)((T + kC - 1) / kC) * kFRecBytes;
  if (dtype != Q35_BF16) return 0;
  const size_t NP = (size_t)((T + kP - 1) / kP);
  return (size_t)B * H * NP * kRecBytes;
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
  if (B > 65535 || H > 65535 || H * B > (1 << 26) || T > ((int64_t)1 << 30) / (H > Hk ? H : Hk))
    return Q35_EUNSUPPORTED;
  // the bf16 scan's output buffer resource spans one row's [T, H, 128] block, addressed with 32-bit byte offsets
  if (dtype == Q35_BF16 && T * H * kD * 2 >= ((int64_t)1 << 31)) return Q35_EUNSUPPORTED;
  if (dtype != Q35_F32 && dtype != Q35_BF16) return Q35_EUNSUPPORTED;
  const size_t need = q35_gdn_chunk_workspace_bytes(B, T, H, Dk, Dv, chunk_size, dtype);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255)) return Q35_EWORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (dtype == Q35_F32) {
    // fp32 inputs: the fp32 WY path (chunk records, then the per-slice scan)
    const int64_t NC = (T + kC - 1) / kC;
    if (NC > 65535) return Q35_EUNSUPPORTED;
    const GdnFront none{};
    hipLaunchKernelGGL(gdn_f32_prep_kernel<false>, dim3((unsigned)NC, (unsigned)H, (unsigned)B), dim3(256), 0, st,
                       (const float*)q, (const float*)k, (const float*)v, g, beta, ws, (int)T, (int)NC, (int)Hk,
                       (int)H, scale, use_qk_l2norm, none);
    gdn_f32_scan_launch(ws, initial_state, final_state, (float*)out, (int)T, (int)NC, (int)H, (int)B, (int)Hk, none,
                        st);
  } else {
    const int64_t NP = (T + kP - 1) / kP;
    if (NP > 65535) return Q35_EUNSUPPORTED;
    dim3 g1((unsigned)H, (unsigned)NP, (unsigned)B), g2((unsigned)(16 * H * B));
    hipLaunchKernelGGL(gdn_pair_prep4_kernel, g1, dim3(256), 0, st, (const __bf16*)q, (const __bf16*)k,
                       (const __bf16*)v, g, beta, ws, (int)T, (int)NP, (int)Hk, (int)H, scale, use_qk_l2norm);
    hipLaunchKernelGGL(gdn_pair_scan_kernel, g2, dim3(kScanThreads), 0, st, ws, initial_state, final_state,
                       (__bf16*)out, (int)T, (int)NP, (int)H, (int)B);
  }
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

extern "C" int q35_gdn_chunk_prefill_conv(const float* y, int64_t ldy, const float* conv_w, const float* conv_bias,
                                          float* conv_state, const float* A_log, const float* dt_bias, int64_t b_off,
                                          int64_t a_off, const float* initial_state, float* final_state, float* out,
                                          int64_t B, int64_t T, int64_t Hk, int64_t H, int64_t Dk, int64_t Dv,
                                          int64_t conv_k, float scale, void* workspace, size_t workspace_bytes,
                                          q35_stream_t stream) {
  using namespace q35;
  if (!y || !conv_w || !conv_state || !A_log || !dt_bias || !out) return Q35_EINVAL;
  if (B <= 0 || T <= 0 || Hk <= 0 || H <= 0 || Dk <= 0 || Dv <= 0 || H % Hk != 0 || conv_k < 2) return Q35_EINVAL;
  if (Dk != kD || Dv != kD || conv_k != kFrontK) return Q35_EUNSUPPORTED;
  const int64_t Kd = Hk * kD, C = 2 * Kd + H * kD;
  if (ldy < C || b_off < 0 || a_off < 0 || b_off + H > ldy || a_off + H > ldy) return Q35_EINVAL;
  if ((ldy & 3) || ((uintptr_t)y & 15) || ((uintptr_t)conv_w & 15) || ((uintptr_t)conv_state & 15) ||
      (conv_bias && ((uintptr_t)conv_bias & 15)))
    return Q35_EUNSUPPORTED;
  // the prep kernel addresses a chunk's rows of y with 32-bit offsets: 67 ldy must fit
  if (B > 65535 || H > 65535 || H * B > (1 << 26) || T > ((int64_t)1 << 30) / H || ldy > (1 << 24) ||
      C > (1 << 28))
    return Q35_EUNSUPPORTED;
  const int64_t NC = (T + kC - 1) / kC;
  if (NC > 65535) return Q35_EUNSUPPORTED;
  const size_t need = q35_gdn_chunk_workspace_bytes(B, T, H, Dk, Dv, kC, Q35_F32);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255)) return Q35_EWORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const GdnFront fe{y, ldy, conv_w, conv_bias, conv_state, A_log, dt_bias, (int)b_off, (int)a_off, (int)C, (int)Kd};
  hipLaunchKernelGGL(gdn_f32_prep_kernel<true>, dim3((unsigned)NC, (unsigned)H, (unsigned)B), dim3(256), 0, st,
                     (const float*)nullptr, (const float*)nullptr, (const float*)nullptr, (const float*)nullptr,
                     (const float*)nullptr, ws, (int)T, (int)NC, (int)Hk, (int)H, scale, 1, fe);
  gdn_f32_scan_launch(ws, initial_state, final_state, out, (int)T, (int)NC, (int)H, (int)B, (int)Hk, fe, st);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
