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
// plain global -> LDS copies. From the fused projection output (q35_gated_attn_prefill_proj) it is also the front
// end: q and k normalised and rotated, k and v appended to the KV cache, q written rotated for the main kernel.
// Inside each group of 16 keys, V^T stores keys in the order 0-3, 8-11, 4-7, 12-15 (bits 2 and 3 of the key index
// swapped): that is the key order in which an MFMA accumulator tile of scores is fed back as a B operand, so every
// A fragment of V^T is one 16-byte read.
// Kernel 2, attn_prefill_kernel: one block of 4 waves per (32-query block, group of up to 4 query heads sharing a kv
// head, batch row); wave w owns query head w of the group, so every K/V tile in LDS serves up to 4 heads. Query
// blocks are issued longest (latest) first. Per 64-key tile each wave computes S^T = K Q^T with 32 x 32 x 16 bf16
// MFMAs (K from LDS, Q^T resident in registers as the B operand: a query's 32 scores sit in one lane pair), the
// online softmax in registers, then O^T += V^T P^T with P^T's accumulator tiles used directly as B operands. Tiles
// arrive by global_load_lds DMA into XOR-swizzled LDS (conflict-free 16-byte operand reads), two stages and one
// barrier per tile (tile kt + 1 is copied while tile kt is computed), each wave copying a quarter of every tile.
#include <atomic>
#include <functional>
#include <mutex>
#include <queue>
#include <type_traits>
#include <vector>

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
// the same with a uniform 64-bit base in SGPRs and a 32-bit per-lane byte offset (the base is moved to SGPRs
// explicitly: the compiler cannot always prove it uniform)
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_dst) {
  const uint64_t a = reinterpret_cast<uint64_t>(sbase);
  const uint64_t u = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_dst), "v"(voff),
               "s"(reinterpret_cast<const void*>(u))
               : "memory", "m0");
}

// a pointer the compiler cannot prove uniform, moved to scalar registers
template <typename T> __device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return reinterpret_cast<T*>(((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
                              (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a));
}

// key order inside a group of 16 keys in V^T (an involution: swaps bits 2 and 3)
__device__ __forceinline__ int vperm(int p) { return (p & 3) | ((p & 4) << 1) | ((p & 8) >> 1); }

// ---------------------------------------------------------------------------------------------------------------
// V^T of one 64-key tile: keys key0 .. key0 + 63 of the rows vrow0 + key * rstride (zero for keys >= nk) into the
// head's V^T block vth [256 dims][Tp keys]. Thread = (8 keys kg, 8 dims dg): an 8 x 8 transpose in registers, each
// dim row written as two 8-byte pieces (keys kg*8 .. +3 and +4 .. +7 land 8 positions apart after the in-group
// permutation).
// Tsrc float: fp32 rows (the fused projection output), rounded to bf16 here; then keys below nold come from the bf16
// rows cold + key * 256 (a KV cache's earlier rows) and key >= nold from row key - nold of vrow0; vcache (when
// given): the values of keys >= nold are also written, as rows, into the cache rows crow0 + key below crows (the
// cache's row stride 256).
template <typename Tsrc>
__device__ __forceinline__ void vt_tile(const Tsrc* __restrict__ vrow0, size_t rstride, int key0, int nk,
                                        __bf16* __restrict__ vth, int Tp, int tid, __bf16* vcache = nullptr,
                                        int crow0 = 0, int crows = 0, const __bf16* cold = nullptr, int nold = 0) {
  const int kg = tid >> 5, dg = tid & 31;
  u32x4 w[8];
  const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = key0 + 8 * kg + i;
    const int kc = min(key, nk - 1);
    u32x4 ld;
    if constexpr (std::is_same<Tsrc, float>::value) {
      if (kc < nold) {
        ld = *reinterpret_cast<const u32x4*>(cold + (size_t)kc * kPD + 8 * dg);
      } else {
        const float* src = vrow0 + (size_t)(kc - nold) * rstride + 8 * dg;
        const f32x4 a = *reinterpret_cast<const f32x4*>(src), c = *reinterpret_cast<const f32x4*>(src + 4);
        const bf16x8 h = {(__bf16)a[0], (__bf16)a[1], (__bf16)a[2], (__bf16)a[3],
                          (__bf16)c[0], (__bf16)c[1], (__bf16)c[2], (__bf16)c[3]};
        ld = __builtin_bit_cast(u32x4, h);
      }
    } else {
      ld = *reinterpret_cast<const u32x4*>(vrow0 + (size_t)kc * rstride + 8 * dg);
    }
    w[i] = key < nk ? ld : z;
    if (vcache && key < nk && key >= nold && crow0 + key < crows)
      *reinterpret_cast<u32x4*>(vcache + (size_t)(crow0 + key) * kPD + 8 * dg) = ld;
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
    __bf16* row = vth + (size_t)d * Tp + key0 + (p0 & ~15);
    *reinterpret_cast<u32x2*>(row + vperm(p0 & 15)) = lo;
    *reinterpret_cast<u32x2*>(row + vperm((p0 & 15) + 4)) = hi;
  }
}

// The attention front end for the form that starts from the fused projection output (q35_gated_attn_prefill_proj;
// the WGSL attnPrep, engine/kernels_qwen35.js:18-69): y [B * T, ldy] fp32 rows of [q | gate] per query head
// (Hq 2 D), then k (Hkv D), then v (Hkv D); q and k normalised with RMS and (1 + w), then rotated. The keys and values
// are also appended to the bf16 caches [B, Hkv, max_len, D] at rows pos0 + t; the queries go, rotated, to
// qr [B, T, Hq, D] bf16.
struct PfFront {
  const float* y;
  int64_t ldy;
  const float* qnw;
  const float* knw;
  float eps;
  __bf16* kc;
  __bf16* vc;
  __bf16* qr;
  int max_len;
};

// ---------------------------------------------------------------------------------------------------------------
// Kernel 1: one block of 256 threads per (64 keys, kv head, row) for the keys and another for the values; with FP
// (the projection-output form, PfFront) also one per (64 tokens, query head of the kv head's group, row) for the
// queries. ROT (rotary dims) is a template parameter so that the rotation pairs are compile-time register indices.
// CACHED (with FP): the call's T tokens sit at cache positions P .. P + T - 1, P = pos_dev[b] clamped to
// 0 .. max_len - T as the cached main kernel clamps it; the keys go to the cache only (the main kernel reads them
// there), and the value blocks cover the cache rows 0 .. P + T - 1 (Tp = max_len): rows below P from the cache, the
// call's rows from y (also appended to the cache).
template <int ROT, bool FP, bool CACHED>
__global__ __launch_bounds__(256) void attn_kv_prep_kernel(const __bf16* __restrict__ k, const __bf16* __restrict__ v,
                                                           const float* __restrict__ cos_t,
                                                           const float* __restrict__ sin_t, int pos0,
                                                           __bf16* __restrict__ kr, __bf16* __restrict__ vt, int T,
                                                           int Tp, int Hkv, int Hq, PfFront fe,
                                                           const int32_t* __restrict__ pos_dev) {
  static_assert(ROT % 16 == 0 && ROT <= kRotMax, "rotary dims");
  static_assert(FP || !CACHED, "the cached form starts from the projection output");
  constexpr int half = ROT / 2;
  const int tid = threadIdx.x;
  // blocks x < ntk prepare the keys of tile x (tokens 64 x ..), the next nvt the values of tile x - ntk, then (FP)
  // the queries: block ntk + nvt + G u + g holds tokens 64 u .. of query head kvh G + g
  const int ntk = CACHED ? (T + kBN - 1) / kBN : Tp / kBN, nvt = Tp / kBN, bx = blockIdx.x;
  const int role = bx < ntk ? 0 : (bx < ntk + nvt ? 1 : 2);  // 0 keys, 1 values, 2 queries
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int G = Hq / Hkv;
  const int key0 = (role == 0 ? bx : role == 1 ? bx - ntk : (bx - ntk - nvt) / G) * kBN;
  const int qh = role == 2 ? kvh * G + (bx - ntk - nvt) % G : 0;
  const size_t head = (size_t)b * Hkv + kvh;
  if constexpr (CACHED) pos0 = min(max(pos_dev[b], 0), Tp - T);
  // Keys and queries: thread = (row r, lane q of 4); a row is 32 segments of 8 dims and thread q takes segments
  // q, q + 4, ... A rotary segment (s < ROT / 8) pairs with the segment half / 8 away; its cos / sin rows are loaded
  // as vectors. Every load of the thread is issued before any is used (one memory round trip per block).
  if (role != 1) {
    constexpr int NSEG = kPD / 8, RS = ROT / 8, HS = half / 8;
    const int r = tid >> 2, q = tid & 3;
    const int key = key0 + r;
    const bool valid = key < T;
    const size_t trow = (size_t)b * T + min(key, T - 1);
    u32x4 w[NSEG / 4], pw[NSEG / 4];
    f32x4 cs[NSEG / 4][2], sn[NSEG / 4][2];
    // FP: the row in fp32 (and its rotation partners), the norm weights of the thread's segments
    f32x4 xf[NSEG / 4][2], pxf[NSEG / 4][2], wf[NSEG / 4][2], pwf[NSEG / 4][2];
    const __bf16* src = k + (trow * Hkv + kvh) * kPD;
    const float* ysrc = nullptr;
    const float* nw = nullptr;
    if constexpr (FP) {
      ysrc = fe.y + trow * fe.ldy + (role == 2 ? (size_t)qh * 2 * kPD : (size_t)Hq * 2 * kPD + (size_t)kvh * kPD);
      nw = role == 2 ? fe.qnw : fe.knw;
    }
#pragma unroll
    for (int i = 0; i < NSEG / 4; ++i) {
      const int sg = q + 4 * i;
      if constexpr (FP) {
        xf[i][0] = *reinterpret_cast<const f32x4*>(ysrc + 8 * sg);
        xf[i][1] = *reinterpret_cast<const f32x4*>(ysrc + 8 * sg + 4);
        wf[i][0] = *reinterpret_cast<const f32x4*>(nw + 8 * sg);
        wf[i][1] = *reinterpret_cast<const f32x4*>(nw + 8 * sg + 4);
      } else {
        w[i] = *reinterpret_cast<const u32x4*>(src + 8 * sg);
      }
      if (4 * i < RS) {  // segments 4 i .. 4 i + 3 may be rotary (compile-time bound)
        const int ps = sg < HS ? sg + HS : sg - HS;
        const int j0 = 8 * (sg < HS ? sg : sg - HS);
        const size_t crow = (size_t)(pos0 + min(key, T - 1)) * half + (sg < RS ? j0 : 0);
        if constexpr (FP) {
          const int pss = sg < RS ? ps : sg;
          pxf[i][0] = *reinterpret_cast<const f32x4*>(ysrc + 8 * pss);
          pxf[i][1] = *reinterpret_cast<const f32x4*>(ysrc + 8 * pss + 4);
          pwf[i][0] = *reinterpret_cast<const f32x4*>(nw + 8 * pss);
          pwf[i][1] = *reinterpret_cast<const f32x4*>(nw + 8 * pss + 4);
        } else {
          pw[i] = *reinterpret_cast<const u32x4*>(src + 8 * (sg < RS ? ps : sg));
        }
        cs[i][0] = *reinterpret_cast<const f32x4*>(cos_t + crow);
        cs[i][1] = *reinterpret_cast<const f32x4*>(cos_t + crow + 4);
        sn[i][0] = *reinterpret_cast<const f32x4*>(sin_t + crow);
        sn[i][1] = *reinterpret_cast<const f32x4*>(sin_t + crow + 4);
      }
    }
    float rr = 1.f;
    if constexpr (FP) {
      // RMS over the row's 256 dims, summed in the order of the one-wave-per-head front end (q35_attn_prep: lane l
      // sums dims 4 l .. 4 l + 3, then a butterfly over lane bits 5 .. 0), so that the cache rows match its bitwise.
      // Here that lane is (i, q, h) = bits 5-3, 2-1, 0: the i levels are local, the q levels the row's 4 threads.
      float s3[2];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        float p[NSEG / 4];
#pragma unroll
        for (int i = 0; i < NSEG / 4; ++i) {
          const f32x4 x = xf[i][h2];
          p[i] = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
        }
        const float s1[4] = {p[0] + p[4], p[1] + p[5], p[2] + p[6], p[3] + p[7]};
        const float s2[2] = {s1[0] + s1[2], s1[1] + s1[3]};
        s3[h2] = s2[0] + s2[1];
        s3[h2] += __shfl_xor(s3[h2], 2, 64);
        s3[h2] += __shfl_xor(s3[h2], 1, 64);
      }
      rr = rsqrtf((s3[0] + s3[1]) * (1.f / kPD) + fe.eps);
    }
    const u32x4 z = {0u, 0u, 0u, 0u};
    // keys: every row of the tile (zero past T; the cached form writes the cache only); queries: the valid rows
    __bf16* dst = role == 2 ? (valid ? fe.qr + (trow * Hq + qh) * kPD : nullptr)
                            : (CACHED ? nullptr : kr + (head * Tp + key) * kPD);
    __bf16* cdst = nullptr;
    if constexpr (FP)
      if (role == 0 && valid && pos0 + key < fe.max_len) cdst = fe.kc + (head * fe.max_len + pos0 + key) * kPD;
#pragma unroll
    for (int i = 0; i < NSEG / 4; ++i) {
      const int sg = q + 4 * i;
      // the segment's 8 values (and, rotary, the partner's), fp32
      float xv[8], yv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (FP) {
          xv[e] = xf[i][e >> 2][e & 3] * rr * (1.f + wf[i][e >> 2][e & 3]);
          yv[e] = (4 * i < RS) ? pxf[i][e >> 2][e & 3] * rr * (1.f + pwf[i][e >> 2][e & 3]) : 0.f;
        } else {
          const uint32_t xw = w[i][e >> 1];
          xv[e] = (e & 1) ? bf16hi(xw) : bf16lo(xw);
          if (4 * i < RS) {
            const uint32_t pwv = pw[i][e >> 1];
            yv[e] = (e & 1) ? bf16hi(pwv) : bf16lo(pwv);
          } else {
            yv[e] = 0.f;
          }
        }
      }
      u32x4 o;
      if (4 * i < RS && sg < RS) {
        const float sgn = sg < HS ? -1.f : 1.f;
        bf16x8 o8;
#pragma unroll
        for (int e = 0; e < 8; ++e) o8[e] = (__bf16)(xv[e] * cs[i][e >> 2][e & 3] + sgn * yv[e] * sn[i][e >> 2][e & 3]);
        o = __builtin_bit_cast(u32x4, o8);
      } else if constexpr (FP) {
        bf16x8 o8;
#pragma unroll
        for (int e = 0; e < 8; ++e) o8[e] = (__bf16)xv[e];
        o = __builtin_bit_cast(u32x4, o8);
      } else {
        o = w[i];
      }
      if (dst) *reinterpret_cast<u32x4*>(dst + 8 * sg) = valid ? o : z;
      if (cdst) *reinterpret_cast<u32x4*>(cdst + 8 * sg) = o;
    }
  } else {
    const float* yv = nullptr;
    if constexpr (FP) yv = fe.y + (size_t)b * T * fe.ldy + (size_t)Hq * 2 * kPD + (size_t)(Hkv + kvh) * kPD;
    if constexpr (CACHED) {
      // cache rows 0 .. pos0 + T - 1; tiles past them are not read by the main kernel
      const int nk = pos0 + T;
      if (key0 >= nk) return;
      __bf16* vch = fe.vc + head * fe.max_len * kPD;
      vt_tile(yv, (size_t)fe.ldy, key0, nk, vt + head * kPD * Tp, Tp, tid, vch, 0, fe.max_len, vch, pos0);
    } else if constexpr (FP) {
      vt_tile(yv, (size_t)fe.ldy, key0, T, vt + head * kPD * Tp, Tp, tid, fe.vc + head * fe.max_len * kPD, pos0,
              fe.max_len);
    } else {
      vt_tile(v + ((size_t)b * T * Hkv + kvh) * kPD, (size_t)Hkv * kPD, key0, T, vt + head * kPD * Tp, Tp, tid);
    }
  }
}

// Cached prefill: V^T of the cache rows a row's queries attend to (keys 0 .. P_b + T - 1, P_b = pos[b]; zero past
// them within the last tile) into the workspace [B, Hkv, D, Tp], Tp the cache length; tiles past them are skipped.
__global__ __launch_bounds__(256) void attn_vcache_prep_kernel(const __bf16* __restrict__ v_cache,
                                                               const int32_t* __restrict__ pos,
                                                               __bf16* __restrict__ vt, int T, int Tp, int Hkv) {
  const int key0 = blockIdx.x * kBN, kvh = blockIdx.y, b = blockIdx.z;
  const int nk = min(max(pos[b], 0), Tp - T) + T;
  if (key0 >= nk) return;
  const size_t head = (size_t)b * Hkv + kvh;
  vt_tile(v_cache + head * Tp * kPD, kPD, key0, nk, vt + head * kPD * Tp, Tp, threadIdx.x);
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
// [Ls, nkt), whose (O, m, l) are combined by attn_prefill_merge_kernel; the others run whole (Ls = 0, every block
// whole and longest first, when the estimate of pf_split_pays finds that faster). Two orders:
// - Independent items, numbered longest first: all first halves (Ls tiles each), then second halves and whole blocks
//   alternately, each in decreasing length, so that the hardware's in-order dispatch to free CUs balances the CUs'
//   total tiles. Used when the items outnumber the CUs.
// - Paired items, used when they fit the device in one wave (one block per CU): the second half of the j-th longest
//   split block (about Ls - j / 2 tiles) and whole block j (about j / 2 + 1 tiles) run one after the other in one
//   block, so every block holds Ls or Ls + 1 tiles. Independent items would leave the short items to a second wave,
//   each paying its query prologue (a memory round trip of several microseconds) on the critical path.
constexpr int kPartFloats = 8192 + 128;  // one wave's partial: O^T [32 x 256] fp32 in accumulator order, m[64], l[64]

struct PfItem {
  int qb, kt0, kt1, half;  // half: -1 for a whole block, else 0 / 1
  int qb2;                 // paired items: the whole block run after this one, else -1
};

__host__ __device__ inline int pf_tiles(int qb) { return (qb * kBQ + kBQ - 1) / kBN + 1; }

__host__ __device__ inline PfItem pf_item(int idx, int nqb, int Ls, bool paired) {
  if (Ls == 0) {
    const int qb = nqb - 1 - idx;
    return {qb, 0, pf_tiles(qb), -1, -1};
  }
  const int qs = 2 * Ls, nsq = nqb - qs;  // blocks qs .. nqb-1 are split
  if (idx < nsq) return {nqb - 1 - idx, 0, Ls, 0, -1};
  if (paired) {
    // j < min(nsq, qs): second half of block nqb-1-j, then whole block j; past that the unpaired remainder (second
    // halves when nsq > qs, else whole blocks nsq .. qs-1)
    const int j = idx - nsq;
    if (j < nsq) return {nqb - 1 - j, Ls, pf_tiles(nqb - 1 - j), 1, j < qs ? j : -1};
    return {j, 0, pf_tiles(j), -1, -1};
  }
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
    return {qb, Ls, pf_tiles(qb), 1, -1};
  }
  const int qb = qs - 1 - p;
  return {qb, 0, pf_tiles(qb), -1, -1};
}

// split length for a launch: none for short sequences, else half of the longest block's tiles
inline int pf_split_len(int nqb) {
  const int nmax = pf_tiles(nqb - 1);
  return nmax >= 8 ? (nmax + 1) / 2 : 0;
}
inline int pf_items(int nqb, int Ls, bool paired) {
  if (Ls == 0) return nqb;
  const int nsq = nqb - 2 * Ls, qs = 2 * Ls;
  return paired ? nsq + (nsq > qs ? nsq : qs) : 2 * nsq + qs;
}

// Estimated end of a launch's blocks (in units of one tile's time) under the hardware's in-order dispatch, each block
// taken by the CU that frees first (one block per CU at a time). A block costs its tiles, 1.5 for its query prologue
// and epilogue, and 0.5 more for a split half's partial stores.
static double pf_dispatch_time(int nqb, int Ls, bool paired, int64_t n_other, int cus) {
  std::priority_queue<double, std::vector<double>, std::greater<double>> free_at;
  for (int c = 0; c < cus; ++c) free_at.push(0.0);
  double end = 0.0;
  const int n = pf_items(nqb, Ls, paired);
  for (int i = 0; i < n; ++i) {
    const PfItem it = pf_item(i, nqb, Ls, paired);
    const double cost = (it.kt1 - it.kt0) + (it.qb2 >= 0 ? pf_tiles(it.qb2) : 0) + 1.5 + (it.half >= 0 ? 0.5 : 0.0);
    for (int64_t o = 0; o < n_other; ++o) {
      const double f = free_at.top() + cost;
      free_at.pop();
      free_at.push(f);
      end = f > end ? f : end;
    }
  }
  return end;
}

// Whether splitting the long query blocks pays on a device of cus CUs: the split schedule's estimated end plus the
// merge kernel (1 for its launch, 0.04 per pair of halves of four waves: the partials' stores and reads) against
// the longest-first order of whole blocks. The costs were fitted to same-box timings of both schedules over ten
// shapes (B 1-4, T 1536-8192, 8 q / 2 kv heads), whose faster schedule they all pick. Decisions are kept per shape.
static bool pf_split_pays(int nqb, int Ls, int64_t n_other, int gw, int cus) {
  if (Ls == 0) return false;
  if (cus <= 0) return true;
  const int64_t nsq = nqb - 2 * Ls;
  // past 256 K blocks (a simulation of about 10 ms) the whole blocks spread evenly however long the longest is
  if ((int64_t)pf_items(nqb, Ls, false) * n_other > ((int64_t)1 << 18)) return false;
  struct Key {
    int nqb, gw, cus;
    int64_t n_other;
  };
  static std::mutex mu;
  static Key keys[32];
  static bool vals[32];
  static int nkeys = 0, next = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < nkeys; ++i)
      if (keys[i].nqb == nqb && keys[i].gw == gw && keys[i].cus == cus && keys[i].n_other == n_other) return vals[i];
  }
  const bool paired = (int64_t)pf_items(nqb, Ls, true) * n_other <= cus;
  const double split = pf_dispatch_time(nqb, Ls, paired, n_other, cus) + 1.0 + 0.01 * gw * (double)(nsq * n_other);
  const bool pays = split < pf_dispatch_time(nqb, 0, false, n_other, cus);
  std::lock_guard<std::mutex> lock(mu);
  keys[next] = Key{nqb, gw, cus, n_other};
  vals[next] = pays;
  next = (next + 1) % 32;
  nkeys = nkeys < 32 ? nkeys + 1 : 32;
  return pays;
}

// GF: the gate is read from the fused projection output (fp32 rows of stride gate_ld, query head h at 2 D h) instead
// of a [B, T, Hq, D] bf16 tensor.
template <int GW, bool PAIRED, bool GF>
__global__ __launch_bounds__(64 * GW, 1) void attn_prefill_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ kr, const __bf16* __restrict__ vt,
    const void* __restrict__ gate, int64_t gate_ld, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    int pos0, __bf16* __restrict__ out, int T, int Tp, int Hq, int Hkv, int ngroups, int rot, float scale, int nqb,
    int B, int Ls, float* __restrict__ part, const int32_t* __restrict__ pos_dev) {
  Q35_ARGS_UPFRONT(q, kr, vt, gate, gate_ld, cos_t, sin_t, pos0, out, T, Tp, Hq, Hkv, ngroups, rot, scale, nqb, B, Ls,
                   part, pos_dev);
  __shared__ PfStage stage[2];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_other = B * Hkv * ngroups;
  const PfItem it0 = pf_item((int)(blockIdx.x / n_other), nqb, Ls, PAIRED);
  const int rem = blockIdx.x % n_other;
  const int b = rem / (Hkv * ngroups);
  const int kvh = (rem / ngroups) % Hkv;
  const int hg = rem % ngroups;
  const int G = Hq / Hkv;
  const int h = kvh * G + hg * GW + wave;
  const int half = rot >> 1;
  const int ln = lane & 31, hh = lane >> 5;
  const size_t head = (size_t)b * Hkv + kvh;
  // uniform bases (scalar registers): the tile copies' addresses are then scalar arithmetic
  const char* kbase = uniform_ptr(reinterpret_cast<const char*>(kr + head * Tp * kPD));
  const char* vbase = uniform_ptr(reinterpret_cast<const char*>(vt + head * kPD * Tp));
  // Cached mode (pos_dev set): the keys are the KV-cache rows 0 .. P + T - 1 of this row, P = pos_dev[b] the
  // position of the call's first token (kr is the cache itself, Tp its length); query t sits at position P + t and
  // attends to keys 0 .. P + t. Otherwise the keys are the call's own T tokens at positions pos0 .. pos0 + T - 1.
  const int qshift = pos_dev ? min(max(pos_dev[b], 0), Tp - T) : 0;
  const int rpos0 = pos_dev ? qshift : pos0;

  // This wave's share of the copies of tile kt into stage s: CPW of the 32 K copies (2 rows each) and CPW of the
  // 32 V^T copies (8 rows each). Copy c of K fills LDS rows 2c, 2c + 1; lane i fetches the 16 bytes that belong at
  // LDS position i: row 2c + hl (hl = i >> 5), logical segment (i & 31) ^ ((2c + hl) & 15). Its source offset is
  // 1024 c + (512 hl + 16 ((i & 31) ^ hl)) ^ 16 ((2c) & 15): one lane constant XOR-ed with a per-copy constant (the
  // XOR only touches bits 5-7). Copy c of V^T fills rows d = 8c + (i >> 3) with logical segment
  // (i & 7) ^ ((d >> 1) & 7) = (i & 7) ^ (i >> 4) ^ 4 (c & 1); its source offset is d 2Tp + 16 segment. The uniform
  // parts go into the scalar base address, so a copy costs one vector XOR.
  constexpr int CPW = 32 / GW;
  const uint32_t kcl = 512 * (lane >> 5) + 16 * ((lane & 31) ^ (lane >> 5));
  const uint32_t vcl = (uint32_t)(lane >> 3) * (uint32_t)(2 * Tp) + 16 * ((lane & 7) ^ (lane >> 4));
  // parts: 1 the K tile, 2 the V^T tile
  auto copy_tile = [&](int kt, int s, int parts) {
    const int key0 = kt * kBN;
    const uint32_t kl = lds_u32(&stage[s].k[0]), vl = lds_u32(&stage[s].v[0]);
    if (parts & 1) {
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int c = CPW * wave + i;  // copy index 0..31
        dma16s(kbase + (size_t)key0 * (kPD * 2) + 1024 * c, kcl ^ (16u * ((2 * c) & 15)),
               __builtin_amdgcn_readfirstlane(kl + 1024 * c));
      }
    }
    if (parts & 2) {
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int c = CPW * wave + i;
        dma16s(vbase + (size_t)8 * c * (Tp * 2) + (size_t)key0 * 2, vcl ^ (64u * (c & 1)),
               __builtin_amdgcn_readfirstlane(vl + 1024 * c));
      }
    }
  };

  // One item (or one segment of a paired item): its query block's tiles kt0 .. kt1 - 1. Inlined once per segment,
  // so each copy is straight-line code with its own register allocation.
  auto run = [&](PfItem it) {
    const int qb = it.qb;
    const int q0 = qb * kBQ;
    // cached mode: the block's key tiles end at its last query's position
    if (pos_dev) it.kt1 = (qshift + min(q0 + kBQ - 1, T - 1)) / kBN + 1;

    // ---- Q^T operand (B of S^T = K Q^T): lane holds query q0 + ln, dims 16 ks + 8 hh + j, rotated. Every load (the
    //      query row, the rotation partners and the cos / sin rows) is issued before the first tile's copies and before
    //      any of them is used, so the prologue costs one memory round trip.
    bf16x8 qop[16];
    {
      const int t = q0 + ln;
      const bool tv = t < T;
      const __bf16* qrow = q + (((size_t)b * T + (tv ? t : T - 1)) * Hq + h) * kPD;
      const int pos = rpos0 + (tv ? t : T - 1);
      u32x4 raw[16];
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) raw[ks] = *reinterpret_cast<const u32x4*>(qrow + 16 * ks + 8 * hh);
      const int nrk = rot >> 4;  // K steps holding rotary dims (rot is a multiple of 16, at most 64)
      u32x4 praw[4];
      f32x4 cs[4][2], sn[4][2];
      if (nrk > 0) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          if (ks < nrk) {
            const int d = 16 * ks + 8 * hh;
            const int pd = d < half ? d + half : d - half;
            const int j0 = d < half ? d : d - half;
            praw[ks] = *reinterpret_cast<const u32x4*>(qrow + pd);
            const float* cp = cos_t + (size_t)pos * half + j0;
            const float* sp = sin_t + (size_t)pos * half + j0;
            cs[ks][0] = *reinterpret_cast<const f32x4*>(cp);
            cs[ks][1] = *reinterpret_cast<const f32x4*>(cp + 4);
            sn[ks][0] = *reinterpret_cast<const f32x4*>(sp);
            sn[ks][1] = *reinterpret_cast<const f32x4*>(sp + 4);
          }
        }
      }
      copy_tile(it.kt0, it.kt0 & 1, 3);
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) {
        const u32x4 r = raw[ks];
        float x[8] = {bf16lo(r[0]), bf16hi(r[0]), bf16lo(r[1]), bf16hi(r[1]),
                      bf16lo(r[2]), bf16hi(r[2]), bf16lo(r[3]), bf16hi(r[3])};
        if (ks < 4 && ks < nrk) {
          const int d = 16 * ks + 8 * hh;
          const u32x4 pr = praw[ks];
          const float y[8] = {bf16lo(pr[0]), bf16hi(pr[0]), bf16lo(pr[1]), bf16hi(pr[1]),
                              bf16lo(pr[2]), bf16hi(pr[2]), bf16lo(pr[3]), bf16hi(pr[3])};
          const float sg = d < half ? -1.f : 1.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float c = cs[ks][j >> 2][j & 3], sv = sn[ks][j >> 2][j & 3];
            x[j] = x[j] * c + sg * y[j] * sv;
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) qop[ks][j] = (__bf16)(tv ? x[j] : 0.f);
      }
    }

    f32x16 o[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) o[mt] = zero16();
    // Scores are kept unscaled; the softmax works in base 2 on scaled scores: p = 2^(s c - m) with c = scale log2(e),
    // m_run the running max of s c.
    const float csc = scale * 1.44269504088896341f;
    float m_run = -INFINITY, l_run = 0.f;
    const int tq = q0 + ln;  // this lane's query
    const int full_tiles = (qshift + q0) / kBN;  // tiles entirely below this block's first query: no mask

    // Per-lane LDS read offsets inside a stage. K: row 32 ksub + ln, logical segment 2 ks + hh, stored at segment
    // (2 ks + hh) ^ (ln & 15): for ks = 8 a + j the offset is ka[j] + 256 a + 16384 ksub. V^T: row 32 mt + ln, logical
    // segment 2 kk + hh stored at (2 kk + hh) ^ ((ln >> 1) & 7): offset va[kk] + 4096 mt.
    int ka[8], va[4];
    {
      const int c2 = (ln >> 1) & 7;
#pragma unroll
      for (int j = 0; j < 8; ++j) ka[j] = 512 * ln + 16 * (hh ^ (ln & 1)) + 32 * (j ^ c2);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) va[kk] = 128 * ln + 16 * ((2 * kk + hh) ^ c2);
    }

    // Raw scores of tile kt into sc (S^T = K Q^T, causally masked with -inf); returns this lane's query's max of the
    // raw scores over the tile's keys.
    auto tile_scores = [&](int kt, f32x16 (&sc)[2]) -> float {
      kt = __builtin_amdgcn_readfirstlane(kt);  // uniform: the tile copies' addresses stay scalar
      const int s = kt & 1;
      // this wave's copies of tile kt are its only ones in flight; after the barrier every wave's have landed and
      // every wave is done with tile kt - 1, whose stage then receives tile kt + 1
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      // tile kt + 1: its K now, its V^T during this tile's accumulation (the two halves of the copy traffic into LDS
      // go with the two phases of the tile)
      if (kt + 1 < it.kt1) copy_tile(kt + 1, s ^ 1, 1);
      const char* kl = reinterpret_cast<const char*>(&stage[s].k[0]);
      // two accumulation chains (one per 32-key half, issued alternately) over four groups of four K steps; the K
      // fragments of group g + 1 are read while the MFMAs of group g run, so LDS latency is hidden behind the matrix
      // core
      f32x16 acc[2] = {zero16(), zero16()};
      auto kread = [&](int g, bf16x8 (&kf)[2][4]) {
#pragma unroll
        for (int ksub = 0; ksub < 2; ++ksub)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int ks = 4 * g + j;
            kf[ksub][j] = *reinterpret_cast<const bf16x8*>(kl + ka[ks & 7] + 256 * (ks >> 3) + 16384 * ksub);
          }
      };
      bf16x8 kfa[2][4], kfb[2][4];
      kread(0, kfa);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x8 (&cur)[2][4] = (g & 1) ? kfb : kfa;
        bf16x8 (&nxt)[2][4] = (g & 1) ? kfa : kfb;
        if (g < 3) kread(g + 1, nxt);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int ksub = 0; ksub < 2; ++ksub)
            acc[ksub] = mfma32(cur[ksub][j], qop[4 * g + j], acc[ksub]);
      }
      // order: reads of group 0; then (reads of g + 1, MFMAs of g) for g = 0..2; then the MFMAs of group 3
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      float mx = -INFINITY;
      if (__builtin_amdgcn_readfirstlane(kt) >= full_tiles) {
        // lane (ln, hh) holds keys 64 kt + 32 ksub + 8 (i >> 2) + 4 hh + (i & 3) of query tq
        const int kl0 = kt * kBN + 4 * hh;
#pragma unroll
        for (int ksub = 0; ksub < 2; ++ksub)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kl0 + 32 * ksub + 8 * (i >> 2) + (i & 3);
            const float x = (key <= tq + qshift && key < T + qshift) ? acc[ksub][i] : -INFINITY;
            sc[ksub][i] = x;
            mx = fmaxf(mx, x);
          }
      } else {
#pragma unroll
        for (int ksub = 0; ksub < 2; ++ksub)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            sc[ksub][i] = acc[ksub][i];
            mx = fmaxf(mx, sc[ksub][i]);
          }
      }
      return fmaxf(mx, __shfl_xor(mx, 32, 64)) * csc;
    };
    // P = 2^(s c - m_run) of tile kt into the row sum, then O^T += V^T P^T: rows = 256 dims (8 tiles of 32), k = 64
    // keys (4 steps of 16). The MFMAs run K step by K step, so those of step kk need only P's group kk: the
    // exponentials of later groups overlap the matrix core.
    auto tile_accumulate = [&](int kt, const f32x16 (&sc)[2]) {
      kt = __builtin_amdgcn_readfirstlane(kt);
      // stage kt + 1 held tile kt - 1, which every wave finished before this tile's barrier
      if (kt + 1 < it.kt1) copy_tile(kt + 1, (kt & 1) ^ 1, 2);
      const char* vl = reinterpret_cast<const char*>(&stage[kt & 1].v[0]);
      auto vread = [&](int kk, bf16x8 (&vf)[8]) {
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) vf[mt] = *reinterpret_cast<const bf16x8*>(vl + va[kk] + 4096 * mt);
      };
      bf16x8 vfa[8], vfb[8];
      vread(0, vfa);
      const float nm = -m_run;
      float ps = 0.f;
      bf16x8 pb[4];
#pragma unroll
      for (int ksub = 0; ksub < 2; ++ksub)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p = __builtin_amdgcn_exp2f(fmaf(sc[ksub][i], csc, nm));
          ps += p;
          pb[2 * ksub + (i >> 3)][i & 7] = (__bf16)p;
        }
      ps += __shfl_xor(ps, 32, 64);
      l_run += ps;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        bf16x8 (&cur)[8] = (kk & 1) ? vfb : vfa;
        bf16x8 (&nxt)[8] = (kk & 1) ? vfa : vfb;
        if (kk < 3) vread(kk + 1, nxt);
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) o[mt] = mfma32(cur[mt], pb[kk], o[mt]);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    };

    // Online softmax along the keys of each lane's query (lane pair l, l ^ 32 holds all 64 keys of a tile). The
    // running max only moves (and O, l are rescaled) when a tile max exceeds it by more than 8 (base 2): p <= 2^8
    // stays exact enough in fp32 and in the bf16 P operand. The inner loop runs the tiles that need no rescale, so O
    // never leaves the MFMA accumulators there; the rescale (a read, multiply and write-back of all 128 accumulator
    // registers) sits outside it and runs a few times per block (always at tile 0). Every lane has a finite score in
    // the first tile of its item (key 0, or a split block's first key, is at or before its query), so m_run is finite
    // from then on.
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
      const float corr = __builtin_amdgcn_exp2f(m_run - mn);
      l_run *= corr;
      m_run = mn;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[mt][i] *= corr;
      tile_accumulate(kt, sc);
      ++kt;
    }

    // ---- a split query block: each half publishes its (O, m, l); attn_prefill_merge_kernel combines them ----
    if (it.half >= 0) {
      const int pair = (qb - 2 * Ls) * n_other + rem;
      float* mine = part + ((size_t)(2 * pair + it.half) * GW + wave) * kPartFloats;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 w = {o[mt][4 * c], o[mt][4 * c + 1], o[mt][4 * c + 2], o[mt][4 * c + 3]};
          *reinterpret_cast<f32x4*>(mine + ((mt * 4 + c) * 64 + lane) * 4) = w;
        }
      mine[8192 + lane] = m_run;
      mine[8192 + 64 + lane] = l_run;
      return;
    }

    // ---- epilogue: normalise, then gate and store whole rows through LDS ----
    // The accumulators hold 16-byte pieces of 32 different query rows; written straight out, every gate load and
    // output store would touch 32 rows. Instead wave w parks its normalised O (32 queries x 256 dims fp32, 32 KB) in
    // bytes 32768 w .. of the stages (free once every wave has left the tile loop), 16-byte segment s of row r at
    // s ^ r, and reads it back by rows: 16 lanes per 512-byte row of gate and output.
    __syncthreads();
    char* ob = reinterpret_cast<char*>(&stage[0]) + 32768 * wave;
    {
      const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 w = {o[mt][4 * c] * inv, o[mt][4 * c + 1] * inv, o[mt][4 * c + 2] * inv,
                           o[mt][4 * c + 3] * inv};
          *reinterpret_cast<f32x4*>(ob + 1024 * ln + 16 * ((8 * mt + 2 * c + hh) ^ ln)) = w;
        }
    }
    __syncthreads();
    {
      const int rs = lane >> 4, g16 = lane & 15;  // row 4 i + rs, dims 16 g16 .. + 15
      u32x4 gr[8][2];
      f32x4 gf[8][4];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int tr = min(q0 + 4 * i + rs, T - 1);
        if constexpr (GF) {
          const float* gp = static_cast<const float*>(gate) + ((size_t)b * T + tr) * gate_ld + (size_t)h * 2 * kPD +
                            16 * g16;
#pragma unroll
          for (int c = 0; c < 4; ++c) gf[i][c] = *reinterpret_cast<const f32x4*>(gp + 4 * c);
        } else {
          const __bf16* gp = static_cast<const __bf16*>(gate) + ((size_t)b * T + tr) * (size_t)Hq * kPD +
                             (size_t)h * kPD + 16 * g16;
          gr[i][0] = *reinterpret_cast<const u32x4*>(gp);
          gr[i][1] = *reinterpret_cast<const u32x4*>(gp + 8);
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 4 * i + rs, tr = q0 + r;
        float x[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 w = *reinterpret_cast<const f32x4*>(ob + 1024 * r + 16 * ((4 * g16 + j) ^ r));
#pragma unroll
          for (int e = 0; e < 4; ++e) x[4 * j + e] = w[e];
        }
        u32x4 ov[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          float gv[8];
          if constexpr (GF) {
#pragma unroll
            for (int e = 0; e < 8; ++e) gv[e] = gf[i][2 * hf + (e >> 2)][e & 3];
          } else {
            const u32x4 gw = gr[i][hf];
            const float gb[8] = {bf16lo(gw[0]), bf16hi(gw[0]), bf16lo(gw[1]), bf16hi(gw[1]),
                                 bf16lo(gw[2]), bf16hi(gw[2]), bf16lo(gw[3]), bf16hi(gw[3])};
#pragma unroll
            for (int e = 0; e < 8; ++e) gv[e] = gb[e];
          }
          bf16x8 pk;
#pragma unroll
          for (int e = 0; e < 8; ++e) pk[e] = (__bf16)(x[8 * hf + e] * sigmoidf_(gv[e]));
          ov[hf] = __builtin_bit_cast(u32x4, pk);
        }
        if (tr < T) {
          __bf16* op = out + ((size_t)b * T + tr) * (size_t)Hq * kPD + (size_t)h * kPD + 16 * g16;
          *reinterpret_cast<u32x4*>(op) = ov[0];
          *reinterpret_cast<u32x4*>(op + 8) = ov[1];
        }
      }
    }
  };

  run(it0);
  if (PAIRED && it0.qb2 >= 0) {
    // every wave is done with the first segment's stages before the second segment's first tile is copied
    __syncthreads();
    run(PfItem{it0.qb2, 0, pf_tiles(it0.qb2), -1, -1});
  }
}

// Kernel 3: the two halves of every split query block. One block of 256 threads per (pair, query head of the group):
// the wave partial is 2048 16-byte chunks in accumulator order (chunk e = (4 mt + c) 64 + l holds dims
// 32 mt + 8 c + 4 (l >> 5) .. + 3 of query q0 + (l & 31)); thread t takes chunks t + 256 j, j < 8, of both halves,
// all loads issued before any is used. The halves are combined in half order, O = O0 2^(m0 - m) + O1 2^(m1 - m), l
// likewise (the result does not depend on which half ran first), then normalised, gated and stored as the main
// kernel's epilogue does. Neither half has a fully masked query: the second half starts at key 64 Ls and every
// query of a split block is at or past it.
// GF: the gate from the fused projection output, as in attn_prefill_kernel.
template <int GW, bool GF>
__global__ __launch_bounds__(256) void attn_prefill_merge_kernel(const float* __restrict__ part,
                                                                 const void* __restrict__ gate, int64_t gate_ld,
                                                                 __bf16* __restrict__ out, int T, int Hq, int Hkv,
                                                                 int ngroups, int B, int Ls) {
  Q35_ARGS_UPFRONT(part, gate, gate_ld, out, T, Hq, Hkv, ngroups, B, Ls);
  const int pair = blockIdx.x, wave = blockIdx.y, tid = threadIdx.x;
  const int n_other = B * Hkv * ngroups;
  const int qb = 2 * Ls + pair / n_other, rem = pair % n_other;
  const int b = rem / (Hkv * ngroups), kvh = (rem / ngroups) % Hkv, hg = rem % ngroups;
  const int h = kvh * (Hq / Hkv) + hg * GW + wave;
  const float* p0 = part + ((size_t)(2 * pair) * GW + wave) * kPartFloats;
  const float* p1 = part + ((size_t)(2 * pair + 1) * GW + wave) * kPartFloats;
  f32x4 w0[8], w1[8], gf[8];
  u32x2 gr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = tid + 256 * j, l = e & 63, mtc = e >> 6;
    const int tq = min(qb * kBQ + (l & 31), T - 1);
    const int d = 8 * mtc + 4 * (l >> 5);  // 32 mt + 8 c + 4 hh with mtc = 4 mt + c
    w0[j] = *reinterpret_cast<const f32x4*>(p0 + (size_t)e * 4);
    w1[j] = *reinterpret_cast<const f32x4*>(p1 + (size_t)e * 4);
    if constexpr (GF)
      gf[j] = *reinterpret_cast<const f32x4*>(static_cast<const float*>(gate) + ((size_t)b * T + tq) * gate_ld +
                                              (size_t)h * 2 * kPD + d);
    else
      gr[j] = *reinterpret_cast<const u32x2*>(static_cast<const __bf16*>(gate) +
                                              ((size_t)b * T + tq) * (size_t)Hq * kPD + (size_t)h * kPD + d);
  }
  // every chunk of thread t has lane l = t & 63 (256 j is a multiple of 64)
  const int l = tid & 63;
  const float m0 = p0[8192 + l], l0 = p0[8192 + 64 + l];
  const float m1 = p1[8192 + l], l1 = p1[8192 + 64 + l];
  const float mm = fmaxf(m0, m1);
  const float c0 = __builtin_amdgcn_exp2f(m0 - mm), c1 = __builtin_amdgcn_exp2f(m1 - mm);
  const float lt = fmaf(l0, c0, l1 * c1);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  const int tq = qb * kBQ + (l & 31);
  if (tq >= T) return;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = tid + 256 * j, mtc = e >> 6;
    const int d = 8 * mtc + 4 * (l >> 5);
    float gv[4];
    if constexpr (GF) {
#pragma unroll
      for (int q = 0; q < 4; ++q) gv[q] = gf[j][q];
    } else {
      gv[0] = bf16lo(gr[j][0]);
      gv[1] = bf16hi(gr[j][0]);
      gv[2] = bf16lo(gr[j][1]);
      gv[3] = bf16hi(gr[j][1]);
    }
    bf16x4 ov;
#pragma unroll
    for (int q = 0; q < 4; ++q) ov[q] = (__bf16)(fmaf(w0[j][q], c0, w1[j][q] * c1) * inv * sigmoidf_(gv[q]));
    *reinterpret_cast<bf16x4*>(out + ((size_t)b * T + tq) * (size_t)Hq * kPD + (size_t)h * kPD + d) = ov;
  }
}

static int64_t padded_T(int64_t T) { return (T + kBN - 1) / kBN * kBN; }

// Compute units of the current device, queried once per device (the paired work order needs every block resident).
static int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Workspace: K rotated and V transposed ([B, Hkv, Tp, D] bf16 each), for the projection-output form the rotated
// queries ([B, T, Hq, D] bf16), then the split blocks' partials ([pairs][2 halves][wave] x kPartFloats fp32).
struct PfLayout {
  size_t q_off, part_off, total;
  int64_t npairs;
};
// Ls: the split length (the workspace functions size for pf_split_len, the most a launch can use).
static PfLayout pf_layout(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, bool fp, int Ls) {
  const int64_t Tp = padded_T(T);
  const int64_t G = Hq / Hkv;
  const int64_t GW = G > 4 ? 4 : G;
  const int64_t nqb = (T + kBQ - 1) / kBQ;
  const int64_t nsq = Ls ? nqb - 2 * Ls : 0;
  PfLayout l;
  l.npairs = nsq * B * Hkv * (G / GW);
  l.q_off = (size_t)2 * B * Hkv * Tp * kPD * sizeof(__bf16);
  l.part_off = l.q_off + (fp ? ((size_t)B * T * Hq * kPD * sizeof(__bf16) + 255) / 256 * 256 : 0);
  l.total = (l.part_off + (size_t)2 * l.npairs * GW * kPartFloats * sizeof(float) + 255) / 256 * 256;
  return l;
}

// Size limits shared by both forms of the own-keys prefill (Q35_OK, or the status to return).
static int pf_check(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t rot) {
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || Hq % Hkv != 0 || rot < 0 || rot > D) return Q35_EINVAL;
  if (D != kPD || (rot % 16) != 0 || rot > kRotMax) return Q35_EUNSUPPORTED;
  const int64_t G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return Q35_EUNSUPPORTED;
  if (T > ((int64_t)1 << 30) || B > 65535 || Hkv > 65535 || T * Hq * D > ((int64_t)1 << 40)) return Q35_EUNSUPPORTED;
  // V^T rows are addressed with 32-bit byte offsets inside a head's [D, Tp] block
  if (padded_T(T) * kPD * 2 >= ((int64_t)1 << 31)) return Q35_EUNSUPPORTED;
  // the pre-pass grid: (2 + G) tiles of 64 per kv head in x
  if ((2 + G) * (padded_T(T) / kBN) > 0x7fffffff) return Q35_EUNSUPPORTED;
  return Q35_OK;
}

// The own-keys prefill (validated arguments): the pre-pass, the main kernel and, for split blocks, the merge.
// FP: q, k and v come from the projection output (fe); gate then points at y + D with row stride gate_ld.
template <bool FP>
static int pf_launch(const void* q, const void* k, const void* v, const void* gate, int64_t gate_ld, const PfFront& fe0,
                     const float* cos, const float* sin, int64_t pos0, void* out, int64_t B, int64_t T, int64_t Hq,
                     int64_t Hkv, int64_t rot, float scale, void* workspace, size_t workspace_bytes,
                     hipStream_t st) {
  const int64_t G = Hq / Hkv;
  const int GW = G > 4 ? 4 : (int)G;
  const int ngroups = (int)(G / GW);
  const int64_t Tp = padded_T(T);
  const int64_t nqb = (T + kBQ - 1) / kBQ;
  const int Lmax = pf_split_len((int)nqb);
  const int64_t n_other = B * Hkv * ngroups;
  if ((int64_t)pf_items((int)nqb, Lmax, false) * n_other > 0x7fffffff) return Q35_EUNSUPPORTED;
  if (pf_layout(B, T, Hq, Hkv, FP, Lmax).npairs > 0x7fffffff) return Q35_EUNSUPPORTED;
  // the workspace as the size functions report it (the split case), checked before any HIP call
  if (!workspace || workspace_bytes < pf_layout(B, T, Hq, Hkv, FP, Lmax).total || ((uintptr_t)workspace & 255))
    return Q35_EWORKSPACE;
  // the first HIP call: the device's compute units decide the split and the work order
  const int cus = device_cus();
  const int Ls = pf_split_pays((int)nqb, Lmax, n_other, GW, cus) ? Lmax : 0;
  const PfLayout lay = pf_layout(B, T, Hq, Hkv, FP, Ls);
  const bool paired = Ls > 0 && (int64_t)pf_items((int)nqb, Ls, true) * n_other <= cus;
  const int64_t nblocks = (int64_t)pf_items((int)nqb, Ls, paired) * n_other;
  char* ws = static_cast<char*>(workspace);
  __bf16* kr = reinterpret_cast<__bf16*>(ws);
  __bf16* vt = kr + (size_t)B * Hkv * Tp * kPD;
  float* part = reinterpret_cast<float*>(ws + lay.part_off);
  PfFront fe = fe0;
  if constexpr (FP) {
    fe.qr = reinterpret_cast<__bf16*>(ws + lay.q_off);
    q = fe.qr;
  }
  const dim3 gp((unsigned)((FP ? 2 + G : 2) * (Tp / kBN)), (unsigned)Hkv, (unsigned)B);
#define Q35_KV_LAUNCH(R)                                                                                        \
  hipLaunchKernelGGL((attn_kv_prep_kernel<R, FP, false>), gp, dim3(256), 0, st, (const __bf16*)k, (const __bf16*)v,  \
                     cos, sin, (int)pos0, kr, vt, (int)T, (int)Tp, (int)Hkv, (int)Hq, fe, (const int32_t*)nullptr)
  switch (rot) {
    case 0: Q35_KV_LAUNCH(0); break;
    case 16: Q35_KV_LAUNCH(16); break;
    case 32: Q35_KV_LAUNCH(32); break;
    case 48: Q35_KV_LAUNCH(48); break;
    default: Q35_KV_LAUNCH(64); break;
  }
#undef Q35_KV_LAUNCH
  // the projection-output form's queries are rotated by the pre-pass: the main kernel then rotates nothing
  const int mrot = FP ? 0 : (int)rot;
#define Q35_PF_LAUNCH(GG)                                                                                           \
  hipLaunchKernelGGL((paired ? attn_prefill_kernel<GG, true, FP> : attn_prefill_kernel<GG, false, FP>),            \
                     dim3((unsigned)nblocks), dim3(64 * GG), 0, st, (const __bf16*)q, kr, vt, gate, gate_ld, cos, sin, \
                     (int)pos0, (__bf16*)out, (int)T, (int)Tp, (int)Hq, (int)Hkv, ngroups, mrot, scale, (int)nqb,     \
                     (int)B, Ls, part, (const int32_t*)nullptr);                                                    \
  if (lay.npairs > 0)                                                                                               \
    hipLaunchKernelGGL((attn_prefill_merge_kernel<GG, FP>), dim3((unsigned)lay.npairs, GG), dim3(256), 0, st, part,  \
                       gate, gate_ld, (__bf16*)out, (int)T, (int)Hq, (int)Hkv, ngroups, (int)B, Ls)
  switch (GW) {
    case 1: Q35_PF_LAUNCH(1); break;
    case 2: Q35_PF_LAUNCH(2); break;
    default: Q35_PF_LAUNCH(4); break;
  }
#undef Q35_PF_LAUNCH
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

}  // namespace q35

extern "C" size_t q35_gated_attn_prefill_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D) {
  using namespace q35;
  if (pf_check(B, T, Hq, Hkv, D, 0) != Q35_OK) return 0;
  return pf_layout(B, T, Hq, Hkv, false, pf_split_len((int)((T + kBQ - 1) / kBQ))).total;
}

extern "C" int q35_gated_attn_prefill(const void* q, const void* k, const void* v, const void* gate,
                                      const float* cos, const float* sin, int64_t pos0, void* out, int64_t B,
                                      int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t rot, float scale,
                                      void* workspace, size_t workspace_bytes, q35_stream_t stream) {
  using namespace q35;
  if (!q || !k || !v || !gate || !out) return Q35_EINVAL;
  if (pos0 < 0 || (rot > 0 && (!cos || !sin))) return Q35_EINVAL;
  const int chk = pf_check(B, T, Hq, Hkv, D, rot);
  if (chk != Q35_OK) return chk;
  return pf_launch<false>(q, k, v, gate, Hq * kPD, PfFront{}, cos, sin, pos0, out, B, T, Hq, Hkv, rot, scale,
                          workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" size_t q35_gated_attn_prefill_proj_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                                                              int64_t D) {
  using namespace q35;
  if (pf_check(B, T, Hq, Hkv, D, 0) != Q35_OK) return 0;
  return pf_layout(B, T, Hq, Hkv, true, pf_split_len((int)((T + kBQ - 1) / kBQ))).total;
}

extern "C" int q35_gated_attn_prefill_proj(const float* y, int64_t ldy, const float* q_norm_w,
                                           const float* k_norm_w, float eps, void* k_cache, void* v_cache,
                                           int64_t pos0, const float* cos, const float* sin, void* out, int64_t B,
                                           int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len,
                                           int64_t rot, float scale, void* workspace, size_t workspace_bytes,
                                           q35_stream_t stream) {
  using namespace q35;
  if (!y || !q_norm_w || !k_norm_w || !k_cache || !v_cache || !out) return Q35_EINVAL;
  if (pos0 < 0 || (rot > 0 && (!cos || !sin))) return Q35_EINVAL;
  const int chk = pf_check(B, T, Hq, Hkv, D, rot);
  if (chk != Q35_OK) return chk;
  if (max_len <= 0 || pos0 + T > max_len || ldy < 2 * Hq * D + 2 * Hkv * D) return Q35_EINVAL;
  if ((ldy & 3) || (((uintptr_t)y | (uintptr_t)q_norm_w | (uintptr_t)k_norm_w) & 15)) return Q35_EUNSUPPORTED;
  if (max_len > 0x7fffffff || B * Hkv * max_len * D > ((int64_t)1 << 40)) return Q35_EUNSUPPORTED;
  PfFront fe{y, ldy, q_norm_w, k_norm_w, eps, (__bf16*)k_cache, (__bf16*)v_cache, nullptr, (int)max_len};
  return pf_launch<true>(nullptr, nullptr, nullptr, y + kPD, ldy, fe, cos, sin, pos0, out, B, T, Hq, Hkv, rot, scale,
                         workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" size_t q35_gated_attn_prefill_cached_workspace_bytes(int64_t B, int64_t Hkv, int64_t D, int64_t max_len) {
  using namespace q35;
  if (B <= 0 || Hkv <= 0 || D != kPD || max_len <= 0 || max_len % kBN != 0) return 0;
  return ((size_t)B * Hkv * q35::kPD * max_len * sizeof(__bf16) + 255) / 256 * 256;
}

extern "C" int q35_gated_attn_prefill_cached(const void* q, const void* k_cache, const void* v_cache,
                                             const void* gate, const int32_t* pos, const float* cos,
                                             const float* sin, void* out, int64_t B, int64_t T, int64_t Hq,
                                             int64_t Hkv, int64_t D, int64_t max_len, int64_t rot, float scale,
                                             void* workspace, size_t workspace_bytes, q35_stream_t stream) {
  using namespace q35;
  if (!q || !k_cache || !v_cache || !gate || !pos || !out) return Q35_EINVAL;
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_len <= 0 || Hq % Hkv != 0 || rot < 0 || rot > D ||
      T > max_len)
    return Q35_EINVAL;
  if (rot > 0 && (!cos || !sin)) return Q35_EINVAL;
  if (D != kPD || (rot % 16) != 0 || rot > kRotMax || max_len % kBN != 0) return Q35_EUNSUPPORTED;
  const int64_t G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return Q35_EUNSUPPORTED;
  const int GW = G > 4 ? 4 : (int)G;
  const int ngroups = (int)(G / GW);
  if (max_len > ((int64_t)1 << 30) || B > 65535 || Hkv > 65535 || T * Hq * D > ((int64_t)1 << 40))
    return Q35_EUNSUPPORTED;
  // V^T rows and cache key rows are addressed with 32-bit byte offsets inside a head's block
  if (max_len * kPD * 2 >= ((int64_t)1 << 31)) return Q35_EUNSUPPORTED;
  const int64_t nqb = (T + kBQ - 1) / kBQ;
  const int64_t nblocks = nqb * B * Hkv * ngroups;
  if (nblocks > 0x7fffffff) return Q35_EUNSUPPORTED;
  const size_t need = q35_gated_attn_prefill_cached_workspace_bytes(B, Hkv, D, max_len);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255)) return Q35_EWORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  __bf16* vt = static_cast<__bf16*>(workspace);
  hipLaunchKernelGGL(attn_vcache_prep_kernel, dim3((unsigned)(max_len / kBN), (unsigned)Hkv, (unsigned)B), dim3(256),
                     0, st, (const __bf16*)v_cache, pos, vt, (int)T, (int)max_len, (int)Hkv);
  // one item per query block (no key split: the key range depends on the device positions), latest block first
#define Q35_PFC_LAUNCH(GG)                                                                                        \
  hipLaunchKernelGGL((attn_prefill_kernel<GG, false, false>), dim3((unsigned)nblocks), dim3(64 * GG), 0, st,     \
                     (const __bf16*)q, (const __bf16*)k_cache, vt, gate, Hq * kPD, cos, sin, 0, (__bf16*)out,      \
                     (int)T, (int)max_len, (int)Hq, (int)Hkv, ngroups, (int)rot, scale, (int)nqb, (int)B, 0,        \
                     (float*)nullptr, pos)
  switch (GW) {
    case 1: Q35_PFC_LAUNCH(1); break;
    case 2: Q35_PFC_LAUNCH(2); break;
    default: Q35_PFC_LAUNCH(4); break;
  }
#undef Q35_PFC_LAUNCH
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

// The cached multi-token form from the fused projection output: workspace V^T [B, Hkv, D, max_len] bf16, then the
// rotated queries [B, T, Hq, D] bf16.
static size_t pfc_proj_q_off(int64_t B, int64_t Hkv, int64_t max_len) {
  return ((size_t)B * Hkv * q35::kPD * max_len * sizeof(__bf16) + 255) / 256 * 256;
}

extern "C" size_t q35_gated_attn_prefill_cached_proj_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                                                                     int64_t D, int64_t max_len) {
  using namespace q35;
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D != kPD || max_len <= 0 || max_len % kBN != 0 ||
      T > max_len)
    return 0;
  const int64_t G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return 0;
  if (max_len > ((int64_t)1 << 30) || B * Hq > ((int64_t)1 << 30)) return 0;
  return pfc_proj_q_off(B, Hkv, max_len) + ((size_t)B * T * Hq * kPD * sizeof(__bf16) + 255) / 256 * 256;
}

extern "C" int q35_gated_attn_prefill_cached_proj(const float* y, int64_t ldy, const float* q_norm_w,
                                                  const float* k_norm_w, float eps, void* k_cache, void* v_cache,
                                                  const int32_t* pos, const float* cos, const float* sin, void* out,
                                                  int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                                  int64_t max_len, int64_t rot, float scale, void* workspace,
                                                  size_t workspace_bytes, q35_stream_t stream) {
  using namespace q35;
  if (!y || !q_norm_w || !k_norm_w || !k_cache || !v_cache || !pos || !out) return Q35_EINVAL;
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_len <= 0 || Hq % Hkv != 0 || rot < 0 || rot > D ||
      T > max_len)
    return Q35_EINVAL;
  if (rot > 0 && (!cos || !sin)) return Q35_EINVAL;
  if (ldy < 2 * Hq * D + 2 * Hkv * D) return Q35_EINVAL;
  if (D != kPD || (rot % 16) != 0 || rot > kRotMax || max_len % kBN != 0) return Q35_EUNSUPPORTED;
  if ((ldy & 3) || (((uintptr_t)y | (uintptr_t)q_norm_w | (uintptr_t)k_norm_w) & 15)) return Q35_EUNSUPPORTED;
  const int64_t G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return Q35_EUNSUPPORTED;
  const int GW = G > 4 ? 4 : (int)G;
  const int ngroups = (int)(G / GW);
  if (max_len > ((int64_t)1 << 30) || B > 65535 || Hkv > 65535 || T * Hq * D > ((int64_t)1 << 40) ||
      B * Hkv * max_len * D > ((int64_t)1 << 40))
    return Q35_EUNSUPPORTED;
  // V^T rows and cache key rows are addressed with 32-bit byte offsets inside a head's block
  if (max_len * kPD * 2 >= ((int64_t)1 << 31)) return Q35_EUNSUPPORTED;
  const int64_t nqb = (T + kBQ - 1) / kBQ, ntk = (T + kBN - 1) / kBN;
  const int64_t nblocks = nqb * B * Hkv * ngroups;
  if (nblocks > 0x7fffffff || ntk * (1 + G) + max_len / kBN > 0x7fffffff) return Q35_EUNSUPPORTED;
  const size_t need = q35_gated_attn_prefill_cached_proj_workspace_bytes(B, T, Hq, Hkv, D, max_len);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255)) return Q35_EWORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  __bf16* vt = static_cast<__bf16*>(workspace);
  __bf16* qr = reinterpret_cast<__bf16*>(static_cast<char*>(workspace) + pfc_proj_q_off(B, Hkv, max_len));
  const PfFront fe{y, ldy, q_norm_w, k_norm_w, eps, (__bf16*)k_cache, (__bf16*)v_cache, qr, (int)max_len};
  const dim3 gp((unsigned)(ntk * (1 + G) + max_len / kBN), (unsigned)Hkv, (unsigned)B);
#define Q35_KVC_LAUNCH(R)                                                                                        \
  hipLaunchKernelGGL((attn_kv_prep_kernel<R, true, true>), gp, dim3(256), 0, st, (const __bf16*)nullptr,          \
                     (const __bf16*)nullptr, cos, sin, 0, (__bf16*)nullptr, vt, (int)T, (int)max_len, (int)Hkv,   \
                     (int)Hq, fe, pos)
  switch (rot) {
    case 0: Q35_KVC_LAUNCH(0); break;
    case 16: Q35_KVC_LAUNCH(16); break;
    case 32: Q35_KVC_LAUNCH(32); break;
    case 48: Q35_KVC_LAUNCH(48); break;
    default: Q35_KVC_LAUNCH(64); break;
  }
#undef Q35_KVC_LAUNCH
  // the queries arrive rotated (rot 0 in the main kernel); keys from the cache, the gate from y
#define Q35_PFCP_LAUNCH(GG)                                                                                        \
  hipLaunchKernelGGL((attn_prefill_kernel<GG, false, true>), dim3((unsigned)nblocks), dim3(64 * GG), 0, st,        \
                     (const __bf16*)qr, (const __bf16*)k_cache, vt, (const void*)(y + kPD), ldy, cos, sin, 0,      \
                     (__bf16*)out, (int)T, (int)max_len, (int)Hq, (int)Hkv, ngroups, 0, scale, (int)nqb, (int)B, 0, \
                     (float*)nullptr, pos)
  switch (GW) {
    case 1: Q35_PFCP_LAUNCH(1); break;
    case 2: Q35_PFCP_LAUNCH(2); break;
    default: Q35_PFCP_LAUNCH(4); break;
  }
#undef Q35_PFCP_LAUNCH
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
