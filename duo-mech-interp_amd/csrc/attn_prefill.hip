// Gated causal GQA attention prefill with partial RoPE and the sigmoid output gate fused (flash-style, MFMA bf16).
//
// Semantics (HF:656-698, eager_attention_forward HF:604-626, apply_rotary_pos_emb HF:554-589; WGSL
// engine/kernels_qwen35.js:50-59 and :73-123):
//   q, k  <- partial RoPE on dims [0, rot): x * cos + rotate_half(x) * sin, pairs (i, i + rot/2), position pos0 + t
//   o_h    = softmax(q_h K^T * scale + causal mask) V     (fp32 softmax; kv head h / (Hq / Hkv))
//   out    = o * sigmoid(gate)
//
// Kernel 1, attn_kv_prep_kernel: K rotated once ([B, Hkv, Tp, D] bf16, keys padded to a multiple of 64 with zeros)
// and V transposed once ([B, Hkv, D, Tp] bf16) into the workspace, so that the main loop stages its tiles with
// plain global -> LDS copies. Inside each group of 16 keys, V^T stores keys in the order 0-3, 8-11, 4-7, 12-15
// (bits 2 and 3 of the key index swapped): that is the key order in which an MFMA accumulator tile of scores is fed
// back as a B operand, so every A fragment of V^T is one 16-byte read.
// Kernel 2, attn_prefill_kernel: one block of 4 waves per (32-query block, group of up to 4 query heads sharing a kv
// head, batch row); wave w owns query head w of the group, so every K/V tile in LDS serves up to 4 heads. Query
// blocks are issued longest (latest) first. Per 64-key tile each wave computes S^T = K Q^T with 32 x 32 x 16 bf16
// MFMAs (K from LDS, Q^T resident in registers as the B operand: a query's 32 scores sit in one lane pair), the
// online softmax in registers, then O^T += V^T P^T with P^T's accumulator tiles used directly as B operands. Tiles
// arrive by global_load_lds DMA into XOR-swizzled LDS (conflict-free 16-byte operand reads), two stages and one
// barrier per tile (tile kt + 1 is copied while tile kt is computed), each wave copying a quarter of every tile.
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kPD = 256;           // head dim
constexpr int kBQ = 32;            // queries per wave
constexpr int kBN = 64;            // keys per tile
constexpr int kRotMax = 64;        // rotary dims supported (Qwen3.5: 64)

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// 16 bytes per lane from global to LDS (lane i's bytes land at M0 + 16 i); no registers are involved. Issued from
// inline asm so the compiler does not order LDS reads behind it; completion is awaited with explicit vmcnt counts.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_dst) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_dst), "v"(src) : "memory", "m0");
}

// key order inside a group of 16 keys in V^T (an involution: swaps bits 2 and 3)
__device__ __forceinline__ int vperm(int p) { return (p & 3) | ((p & 4) << 1) | ((p & 8) >> 1); }

// ---------------------------------------------------------------------------------------------------------------
// Kernel 1: one block of 256 threads per (64 keys, kv head, row). ROT (rotary dims) is a template parameter so that
// the rotation pairs are compile-time register indices.
template <int ROT>
__global__ __launch_bounds__(256) void attn_kv_prep_kernel(const __bf16* __restrict__ k, const __bf16* __restrict__ v,
                                                           const float* __restrict__ cos_t,
                                                           const float* __restrict__ sin_t, int pos0,
                                                           __bf16* __restrict__ kr, __bf16* __restrict__ vt, int T,
                                                           int Tp, int Hkv, int* __restrict__ cnt, int ncnt) {
  static_assert(ROT % 16 == 0 && ROT <= kRotMax, "rotary dims");
  constexpr int half = ROT / 2;
  const int tid = threadIdx.x;
  // the attention kernel's split-block arrival counters start every launch at zero
  {
    const int lb = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const int nb = gridDim.x * gridDim.y * gridDim.z;
    for (int i = lb * 256 + tid; i < ncnt; i += nb * 256) cnt[i] = 0;
  }
  const int key0 = blockIdx.x * kBN, kvh = blockIdx.y, b = blockIdx.z;
  const size_t head = (size_t)b * Hkv + kvh;
  // K: thread = (row r, quarter cq of the dims); the rotary dims [0, rot) all sit in quarter 0
  {
    const int r = tid >> 2, cq = tid & 3;
    const int key = key0 + r;
    const bool valid = key < T;
    const __bf16* src = k + (((size_t)b * T + min(key, T - 1)) * Hkv + kvh) * kPD + 64 * cq;
    u32x4 w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = *reinterpret_cast<const u32x4*>(src + 8 * i);
    if (ROT > 0 && cq == 0 && valid) {
      float x[64];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[8 * i + 2 * e] = bf16lo(w[i][e]);
          x[8 * i + 2 * e + 1] = bf16hi(w[i][e]);
        }
      const float* cr = cos_t + (size_t)(pos0 + key) * half;
      const float* sr = sin_t + (size_t)(pos0 + key) * half;
      float y[64];
#pragma unroll
      for (int d = 0; d < 64; ++d) {
        if (d < ROT) {
          const int j = d < half ? d : d - half;
          const float pr = d < half ? -x[(d + half) & 63] : x[(d + 64 - half) & 63];
          y[d] = x[d] * cr[j] + pr * sr[j];
        } else {
          y[d] = x[d];
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        bf16x8 o8;
#pragma unroll
        for (int e = 0; e < 8; ++e) o8[e] = (__bf16)y[8 * i + e];
        w[i] = __builtin_bit_cast(u32x4, o8);
      }
    }
    const u32x4 z = {0u, 0u, 0u, 0u};
    __bf16* dst = kr + (head * Tp + key) * kPD + 64 * cq;
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4*>(dst + 8 * i) = valid ? w[i] : z;
  }
  // V^T: thread = (8 keys kg, 8 dims dg); an 8 x 8 transpose in registers, each dim row written as two 8-byte
  // pieces (keys kg*8 .. +3 and +4 .. +7 land 8 positions apart after the in-group permutation)
  {
    const int kg = tid >> 5, dg = tid & 31;
    u32x4 w[8];
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = key0 + 8 * kg + i;
      const u32x4 ld = *reinterpret_cast<const u32x4*>(v + (((size_t)b * T + min(key, T - 1)) * Hkv + kvh) * kPD +
                                                      8 * dg);
      w[i] = key < T ? ld : z;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      auto h16 = [&](const u32x4& r) -> uint32_t {
        const uint32_t x = r[e >> 1];
        return (e & 1) ? (x >> 16) : (x & 0xffffu);
      };
      u32x2 lo, hi;
      lo[0] = h16(w[0]) | (h16(w[1]) << 16);
      lo[1] = h16(w[2]) | (h16(w[3]) << 16);
      hi[0] = h16(w[4]) | (h16(w[5]) << 16);
      hi[1] = h16(w[6]) | (h16(w[7]) << 16);
      const int d = 8 * dg + e;
      const int p0 = 8 * kg;  // first key of this unit inside the tile
      __bf16* row = vt + (head * kPD + d) * Tp + key0 + (p0 & ~15);
      *reinterpret_cast<u32x2*>(row + vperm(p0 & 15)) = lo;
      *reinterpret_cast<u32x2*>(row + vperm((p0 & 15) + 4)) = hi;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Kernel 2. LDS tiles: K [64 keys][512 B], 16-byte segment s of row r at s ^ (r & 15); V^T [256 dims][128 B],
// segment s of row d at s ^ ((d >> 1) & 7). The copies apply the swizzle on the global side (lane i of a copy
// fetches the segment that belongs at LDS position i).
struct PfStage {
  __bf16 k[kBN * kPD];
  __bf16 v[kPD * kBN];
};

// Work items. Query block qb needs key tiles 0 .. nkt(qb) - 1, so the causal blocks range from 1 to ~T/64 tiles. With
// a split length Ls > 0, every block with more than Ls tiles (qb >= 2 Ls) is run as two items, tiles [0, Ls) and
// [Ls, nkt), whose (O, m, l) are merged by whichever finishes second; the others run whole. Items are numbered
// longest first: all first halves (Ls tiles each), then second halves and whole blocks alternately, each in
// decreasing length, so that the hardware's in-order dispatch to free CUs balances the CUs' total tiles.
constexpr int kPartFloats = 8192 + 128;  // one wave's partial: O^T [32 x 256] fp32 in accumulator order, m[64], l[64]

struct PfItem {
  int qb, kt0, kt1, half;  // half: -1 for a whole block, else 0 / 1
};

__host__ __device__ inline int pf_tiles(int qb) { return (qb * kBQ + kBQ - 1) / kBN + 1; }

__host__ __device__ inline PfItem pf_item(int idx, int nqb, int Ls) {
  if (Ls == 0) {
    const int qb = nqb - 1 - idx;
    return {qb, 0, pf_tiles(qb), -1};
  }
  const int qs = 2 * Ls, nsq = nqb - qs;  // blocks qs .. nqb-1 are split
  if (idx < nsq) return {nqb - 1 - idx, 0, Ls, 0};
  const int j = idx - nsq, m2 = nsq < qs ? nsq : qs;
  bool second;
  int p;
  if (j < 2 * m2) {
    p = j >> 1;
    second = (j & 1) == 0;
  } else {
    p = m2 + (j - 2 * m2);
    second = nsq > qs;
  }
  if (second) {
    const int qb = nqb - 1 - p;
    return {qb, Ls, pf_tiles(qb), 1};
  }
  const int qb = qs - 1 - p;
  return {qb, 0, pf_tiles(qb), -1};
}

// split length for a launch: none for short sequences, else half of the longest block's tiles
inline int pf_split_len(int nqb) {
  const int nmax = pf_tiles(nqb - 1);
  return nmax >= 8 ? (nmax + 1) / 2 : 0;
}
inline int pf_items(int nqb, int Ls) { return Ls == 0 ? nqb : 2 * (nqb - 2 * Ls) + 2 * Ls; }

template <int GW>
__global__ __launch_bounds__(64 * GW, 1) void attn_prefill_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ kr, const __bf16* __restrict__ vt,
    const __bf16* __restrict__ gate, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int pos0,
    __bf16* __restrict__ out, int T, int Tp, int Hq, int Hkv, int ngroups, int rot, float scale, int nqb, int B,
    int Ls, float* __restrict__ part, int* __restrict__ cnt) {
  __shared__ PfStage stage[2];
  __shared__ int merge_here;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_other = B * Hkv * ngroups;
  const PfItem it = pf_item((int)(blockIdx.x / n_other), nqb, Ls);
  const int qb = it.qb;
  const int rem = blockIdx.x % n_other;
  const int b = rem / (Hkv * ngroups);
  const int kvh = (rem / ngroups) % Hkv;
  const int hg = rem % ngroups;
  const int G = Hq / Hkv;
  const int h = kvh * G + hg * GW + wave;
  const int q0 = qb * kBQ;
  const int half = rot >> 1;
  const int ln = lane & 31, hh = lane >> 5;
  const size_t head = (size_t)b * Hkv + kvh;
  const char* kbase = reinterpret_cast<const char*>(kr + head * Tp * kPD);
  const char* vbase = reinterpret_cast<const char*>(vt + head * kPD * Tp);

  // this wave's share of the copies of tile kt into stage s: CPW of the 32 K copies (2 rows each) and CPW of the
  // 32 V^T copies (8 rows each)
  constexpr int CPW = 32 / GW;
  auto copy_tile = [&](int kt, int s) {
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));  // keep the per-lane source offsets out of registers between tiles
    const int key0 = kt * kBN;
    const uint32_t kl = lds_u32(&stage[s].k[0]), vl = lds_u32(&stage[s].v[0]);
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int c = CPW * wave + i;  // copy index 0..31
      const int r = 2 * c + (lane >> 5), ps = lane & 31;
      const int ls = ps ^ (r & 15);
      dma16(kbase + (size_t)(key0 + r) * (kPD * 2) + 16 * ls, __builtin_amdgcn_readfirstlane(kl + 1024 * c));
    }
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int c = CPW * wave + i;
      const int d = 8 * c + (lane >> 3), ps = lane & 7;
      const int ls = ps ^ ((d >> 1) & 7);
      dma16(vbase + (size_t)d * (Tp * 2) + (size_t)key0 * 2 + 16 * ls, __builtin_amdgcn_readfirstlane(vl + 1024 * c));
    }
  };

  copy_tile(it.kt0, it.kt0 & 1);
  // ---- Q^T operand (B of S^T = K Q^T): lane holds query q0 + ln, dims 16 ks + 8 hh + j, rotated ----
  bf16x8 qop[16];
  {
    const int t = q0 + ln;
    const bool tv = t < T;
    const __bf16* qrow = q + (((size_t)b * T + (tv ? t : 0)) * Hq + h) * kPD;
    const int pos = pos0 + t;
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      const int d = 16 * ks + 8 * hh;
      const u32x4 raw = *reinterpret_cast<const u32x4*>(qrow + d);
      float x[8] = {bf16lo(raw[0]), bf16hi(raw[0]), bf16lo(raw[1]), bf16hi(raw[1]),
                    bf16lo(raw[2]), bf16hi(raw[2]), bf16lo(raw[3]), bf16hi(raw[3])};
      if (tv && d < rot) {
        const int pd = d < half ? d + half : d - half;
        const u32x4 pr = *reinterpret_cast<const u32x4*>(qrow + pd);
        const float y[8] = {bf16lo(pr[0]), bf16hi(pr[0]), bf16lo(pr[1]), bf16hi(pr[1]),
                            bf16lo(pr[2]), bf16hi(pr[2]), bf16lo(pr[3]), bf16hi(pr[3])};
        const int j0 = d < half ? d : d - half;
        const float sg = d < half ? -1.f : 1.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float c = cos_t[(size_t)pos * half + j0 + j], sn = sin_t[(size_t)pos * half + j0 + j];
          x[j] = x[j] * c + sg * y[j] * sn;
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) qop[ks][j] = (__bf16)(tv ? x[j] : 0.f);
    }
  }

  f32x16 o[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o[mt] = zero16();
  float m_run = -INFINITY, l_run = 0.f;
  const int tq = q0 + ln;  // this lane's query
  const int full_tiles = q0 / kBN;  // tiles entirely below this block's first query: no mask

  // Scores of tile kt (scaled and causally masked) into sc; returns this lane's query's max over the tile's keys.
  auto tile_scores = [&](int kt, f32x16 (&sc)[2]) -> float {
    const int s = kt & 1;
    // this wave's copies of tile kt are its only ones in flight; after the barrier every wave's have landed and
    // every wave is done with tile kt - 1, whose stage then receives tile kt + 1
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kt + 1 < it.kt1) copy_tile(kt + 1, s ^ 1);
    const char* kl = reinterpret_cast<const char*>(&stage[s].k[0]);
    // the operand addresses below are recomputed every tile from an opaque copy of the lane id: hoisted out of the
    // loop they would occupy some 60 registers, and the kernel is register-bound
    int lo_ = threadIdx.x & 63;
    asm volatile("" : "+v"(lo_));
    const int ln = lo_ & 31, hh = lo_ >> 5;
    // S^T = K Q^T for the two 32-key halves of the tile (rows = keys, cols = this wave's 32 queries): four
    // independent accumulation chains, K fragments read four K steps at a time
    f32x16 acc[2][2];
#pragma unroll
    for (int ksub = 0; ksub < 2; ++ksub) { acc[ksub][0] = zero16(); acc[ksub][1] = zero16(); }
#pragma unroll
    for (int ks0 = 0; ks0 < 16; ks0 += 4) {
      bf16x8 kf[2][4];
#pragma unroll
      for (int ksub = 0; ksub < 2; ++ksub) {
        const int r = 32 * ksub + ln;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          kf[ksub][j] = *reinterpret_cast<const bf16x8*>(kl + r * 512 + 16 * ((2 * (ks0 + j) + hh) ^ (r & 15)));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int ksub = 0; ksub < 2; ++ksub) acc[ksub][j & 1] = mfma32(kf[ksub][j], qop[ks0 + j], acc[ksub][j & 1]);
      // all eight reads first, then the eight MFMAs (the default schedule waits on each read pair in turn)
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    }
    float mx = -INFINITY;
    const bool masked = kt >= full_tiles;
#pragma unroll
    for (int ksub = 0; ksub < 2; ++ksub)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kt * kBN + 32 * ksub + 8 * (i >> 2) + 4 * hh + (i & 3);
        float x = (acc[ksub][0][i] + acc[ksub][1][i]) * scale;
        if (masked) x = (key <= tq && key < T) ? x : -INFINITY;
        sc[ksub][i] = x;
        mx = fmaxf(mx, x);
      }
    return fmaxf(mx, __shfl_xor(mx, 32, 64));
  };
  // P = exp(S - m_run) of tile kt into the row sum, then O^T += V^T P^T: rows = 256 dims (8 tiles of 32),
  // k = 64 keys (4 steps of 16); V^T fragments read two dim tiles at a time
  auto tile_accumulate = [&](int kt, const f32x16 (&sc)[2]) {
    const char* vl = reinterpret_cast<const char*>(&stage[kt & 1].v[0]);
    int lo_ = threadIdx.x & 63;
    asm volatile("" : "+v"(lo_));
    const int ln = lo_ & 31, hh = lo_ >> 5;
    float ps = 0.f;
    bf16x8 pb[4];
#pragma unroll
    for (int ksub = 0; ksub < 2; ++ksub)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = __expf(sc[ksub][i] - m_run);
        ps += p;
        pb[2 * ksub + (i >> 3)][i & 7] = (__bf16)p;
      }
    ps += __shfl_xor(ps, 32, 64);
    l_run += ps;
#pragma unroll
    for (int mt0 = 0; mt0 < 8; mt0 += 2) {
      bf16x8 vf[2][4];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int d = 32 * (mt0 + u) + ln;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          vf[u][kk] = *reinterpret_cast<const bf16x8*>(vl + d * 128 + 16 * ((2 * kk + hh) ^ ((d >> 1) & 7)));
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int u = 0; u < 2; ++u) o[mt0 + u] = mfma32(vf[u][kk], pb[kk], o[mt0 + u]);
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    }
  };

  // Online softmax along the keys of each lane's query (lane pair l, l ^ 32 holds all 64 keys of a tile). The
  // running max only moves (and O, l are rescaled) when a tile max exceeds it by more than 8: p = exp(s - m) <= e^8
  // stays exact enough in fp32 and in the bf16 P operand. The inner loop runs the tiles that need no rescale, so O
  // never leaves the MFMA accumulators there; the rescale (a read, multiply and write-back of all 128 accumulator
  // registers) sits outside it and runs a few times per block (always at tile 0).
  int kt = it.kt0;
  while (kt < it.kt1) {
    f32x16 sc[2];
    float mx = tile_scores(kt, sc);
    while (!__any(mx > m_run + 8.f)) {
      tile_accumulate(kt, sc);
      if (++kt == it.kt1) break;
      mx = tile_scores(kt, sc);
    }
    if (kt == it.kt1) break;
    const float mn = fmaxf(m_run, mx);
    const float corr = __expf(m_run - mn);
    l_run *= corr;
    m_run = mn;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[mt][i] *= corr;
    tile_accumulate(kt, sc);
    ++kt;
  }

  // ---- a split query block: both halves publish (O, m, l); the second to finish merges and stores ----
  if (it.half >= 0) {
    const int pair = (qb - 2 * Ls) * n_other + rem;
    float* mine = part + ((size_t)(2 * pair + it.half) * GW + wave) * kPartFloats;
    const float* other = part + ((size_t)(2 * pair + (it.half ^ 1)) * GW + wave) * kPartFloats;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 w = {o[mt][4 * c], o[mt][4 * c + 1], o[mt][4 * c + 2], o[mt][4 * c + 3]};
        *reinterpret_cast<f32x4*>(mine + ((mt * 4 + c) * 64 + lane) * 4) = w;
      }
    mine[8192 + lane] = m_run;
    mine[8192 + 64 + lane] = l_run;
    // release: this block's partial is visible device-wide before its arrival is counted
    __threadfence();
    __syncthreads();
    if (tid == 0) merge_here = atomicAdd(cnt + pair, 1);
    __syncthreads();
    if (merge_here == 0) return;  // the other half is still running and will merge
    __threadfence();              // acquire: the other half's partial was published before its count
    // O = O0 e^(m0 - m) + O1 e^(m1 - m), l likewise, always in half order so that the result does not depend on
    // which half finished last. Neither half has a fully masked query: the second half starts at key 64 Ls and every
    // query of a split block is at or past it.
    const float m_o = other[8192 + lane], l_o = other[8192 + 64 + lane];
    const float m0 = it.half ? m_o : m_run, m1 = it.half ? m_run : m_o;
    const float l0 = it.half ? l_o : l_run, l1 = it.half ? l_run : l_o;
    const float mm = fmaxf(m0, m1);
    const float c0 = __expf(m0 - mm), c1 = __expf(m1 - mm);
    l_run = fmaf(l0, c0, l1 * c1);
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 w = *reinterpret_cast<const f32x4*>(other + ((mt * 4 + c) * 64 + lane) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = o[mt][4 * c + e];
          o[mt][4 * c + e] = it.half ? fmaf(w[e], c0, a * c1) : fmaf(a, c0, w[e] * c1);
        }
      }
  }

  // ---- epilogue: normalise, gate, store ----
  if (tq < T) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    const size_t rowo = ((size_t)b * T + tq) * (size_t)Hq * kPD + (size_t)h * kPD;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = 32 * mt + 8 * c + 4 * hh;
        const u32x2 gr = *reinterpret_cast<const u32x2*>(gate + rowo + d);
        const float gv[4] = {bf16lo(gr[0]), bf16hi(gr[0]), bf16lo(gr[1]), bf16hi(gr[1])};
        bf16x4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (__bf16)(o[mt][4 * c + e] * inv * sigmoidf_(gv[e]));
        *reinterpret_cast<bf16x4*>(out + rowo + d) = ov;
      }
    }
  }
}

static int64_t padded_T(int64_t T) { return (T + kBN - 1) / kBN * kBN; }

// Workspace: K rotated and V transposed ([B, Hkv, Tp, D] bf16 each), then the split blocks' partials
// ([pairs][2 halves][wave] x kPartFloats fp32), then one int arrival counter per pair.
struct PfLayout {
  size_t part_off, cnt_off, total;
  int64_t ncnt;
};
static PfLayout pf_layout(int64_t B, int64_t T, int64_t Hq, int64_t Hkv) {
  const int64_t Tp = padded_T(T);
  const int64_t G = Hq / Hkv;
  const int64_t GW = G > 4 ? 4 : G;
  const int64_t nqb = (T + kBQ - 1) / kBQ;
  const int Ls = pf_split_len((int)nqb);
  const int64_t nsq = Ls ? nqb - 2 * Ls : 0;
  PfLayout l;
  l.ncnt = nsq * B * Hkv * (G / GW);
  l.part_off = (size_t)2 * B * Hkv * Tp * kPD * sizeof(__bf16);
  l.cnt_off = l.part_off + (size_t)2 * l.ncnt * GW * kPartFloats * sizeof(float);
  l.total = (l.cnt_off + (size_t)l.ncnt * sizeof(int) + 255) / 256 * 256;
  return l;
}

}  // namespace q35

extern "C" size_t q35_gated_attn_prefill_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D) {
  using namespace q35;
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D != kPD) return 0;
  const int64_t G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return 0;
  if (T > ((int64_t)1 << 30) || B * Hq > ((int64_t)1 << 30)) return 0;
  return pf_layout(B, T, Hq, Hkv).total;
}

extern "C" int q35_gated_attn_prefill(const void* q, const void* k, const void* v, const void* gate,
                                      const float* cos, const float* sin, int64_t pos0, void* out, int64_t B,
                                      int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t rot, float scale,
                                      void* workspace, size_t workspace_bytes, q35_stream_t stream) {
  using namespace q35;
  if (!q || !k || !v || !gate || !out) return Q35_EINVAL;
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || Hq % Hkv != 0 || rot < 0 || rot > D || pos0 < 0)
    return Q35_EINVAL;
  if (rot > 0 && (!cos || !sin)) return Q35_EINVAL;
  if (D != kPD || (rot % 16) != 0 || rot > kRotMax) return Q35_EUNSUPPORTED;
  const int64_t G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return Q35_EUNSUPPORTED;
  const int GW = G > 4 ? 4 : (int)G;
  const int ngroups = (int)(G / GW);
  const int64_t Tp = padded_T(T);
  if (T > ((int64_t)1 << 30) || B > 65535 || Hkv > 65535 || T * Hq * D > ((int64_t)1 << 40)) return Q35_EUNSUPPORTED;
  const int64_t nqb = (T + kBQ - 1) / kBQ;
  const int Ls = pf_split_len((int)nqb);
  const int64_t nblocks = (int64_t)pf_items((int)nqb, Ls) * B * Hkv * ngroups;
  if (nblocks > 0x7fffffff) return Q35_EUNSUPPORTED;
  // V^T rows are addressed with 32-bit byte offsets inside a head's [D, Tp] block
  if (Tp * kPD * 2 >= ((int64_t)1 << 31)) return Q35_EUNSUPPORTED;
  const PfLayout lay = pf_layout(B, T, Hq, Hkv);
  if (lay.ncnt > 0x7fffffff) return Q35_EUNSUPPORTED;
  if (!workspace || workspace_bytes < lay.total || ((uintptr_t)workspace & 255)) return Q35_EWORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  __bf16* kr = reinterpret_cast<__bf16*>(ws);
  __bf16* vt = kr + (size_t)B * Hkv * Tp * kPD;
  float* part = reinterpret_cast<float*>(ws + lay.part_off);
  int* cnt = reinterpret_cast<int*>(ws + lay.cnt_off);
  const dim3 gp((unsigned)(Tp / kBN), (unsigned)Hkv, (unsigned)B);
#define Q35_KV_LAUNCH(R)                                                                                         \
  hipLaunchKernelGGL(attn_kv_prep_kernel<R>, gp, dim3(256), 0, st, (const __bf16*)k, (const __bf16*)v, cos, sin, \
                     (int)pos0, kr, vt, (int)T, (int)Tp, (int)Hkv, cnt, (int)lay.ncnt)
  switch (rot) {
    case 0: Q35_KV_LAUNCH(0); break;
    case 16: Q35_KV_LAUNCH(16); break;
    case 32: Q35_KV_LAUNCH(32); break;
    case 48: Q35_KV_LAUNCH(48); break;
    default: Q35_KV_LAUNCH(64); break;
  }
#undef Q35_KV_LAUNCH
#define Q35_PF_LAUNCH(GG)                                                                                         \
  hipLaunchKernelGGL(attn_prefill_kernel<GG>, dim3((unsigned)nblocks), dim3(64 * GG), 0, st, (const __bf16*)q,    \
                     kr, vt, (const __bf16*)gate, cos, sin, (int)pos0, (__bf16*)out, (int)T, (int)Tp, (int)Hq,     \
                     (int)Hkv, ngroups, (int)rot, scale, (int)nqb, (int)B, Ls, part, cnt)
  switch (GW) {
    case 1: Q35_PF_LAUNCH(1); break;
    case 2: Q35_PF_LAUNCH(2); break;
    default: Q35_PF_LAUNCH(4); break;
  }
#undef Q35_PF_LAUNCH
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
