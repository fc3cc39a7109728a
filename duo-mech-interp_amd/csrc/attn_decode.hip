// Gated GQA attention decode: one new query token per row over a bf16 KV cache, split-K over the context.
//
// Semantics (HF:656-698 with a cache, eager_attention_forward HF:604-626; WGSL engine/kernels_qwen35.js:73-123):
//   q_h   <- partial RoPE at position cache_len[b] - 1 (pairs (i, i + rot/2) on the first rot dims, HF:554-589)
//   o_h    = softmax(q_h . K^T * scale) V      over keys 0 .. cache_len[b]-1 of kv head h / (Hq / Hkv)
//   out_h  = o_h * sigmoid(gate_h)             (HF:698)
//
// Pass 1 (attn_decode_partial_kernel): one block of 4 waves per (split, kv head, row). The G = Hq / Hkv query heads
// that share a kv head are the M rows of one 16x16x32 MFMA tile, so each K row is read from HBM once for all G
// heads. Each wave walks 16-key tiles of the block's span with the next tile's K and V loads in flight while the
// current tile is computed: scores via 8 MFMAs whose B operand is loaded straight from the cache (16 contiguous
// bytes per lane), an online softmax on the 16 columns with DPP row reductions (no LDS round trips), then P.V on the
// vector ALU with fully coalesced 16-byte V-row loads (32 lanes cover one 512-byte row). The four waves'
// (max, sum, acc) are merged in LDS and written as one partial per (row, kv head, split).
// Pass 2 (attn_decode_merge_kernel): log-sum-exp merge over splits, sigmoid gate, bf16 store; every load of a
// thread is issued before the first is used (one memory round trip).
// HBM traffic is the K and V spans once (AI ~ 4 flop/byte): the kernel is bandwidth bound by design.
//
// From the fused projection output (q35_gated_attn_decode_proj, the WGSL attnPrep + attention for one token,
// engine/kernels_qwen35.js:18-123): the partial kernel reads q from y and normalises it (RMS with 1 + w) before the
// rotation; split 0's block also forms the token's own key (normalised, rotated) and value, appends them to the caches
// at the token's position and folds that key into its partial; the merge reads the gate from y. One launch fewer
// per decode step than the front end followed by the decode, and no q / gate round trip through memory.
#include <atomic>
#include <mutex>

#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kDecD = 256;  // head dim
constexpr int kDecTile = 16;

__device__ __forceinline__ f32x4 unpack_bf16x4(const u32x2& r) {
  f32x4 o = {bf16lo(r.x), bf16hi(r.x), bf16lo(r.y), bf16hi(r.y)};
  return o;
}

// Max / sum over the 16 lanes of a DPP row (lanes 16 r .. 16 r + 15), result in every lane of the row: quad_perm
// [1,0,3,2] and [2,3,0,1] combine the lanes of a quad, row_half_mirror (lane i <- 7 - i within 8) the two quads of
// a half row, row_mirror (lane i <- 15 - i) the two halves.
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  return fmaxf(v, dpp_mov<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  return v + dpp_mov<0x140>(v);
}

// Query source of the partial kernel. FP false: bf16 q [B, Hq, D], the cache holding every key up to and including
// the token's (cache_len[b] keys, the query at position cache_len[b] - 1). FP true: the token's fused projection
// output y (fp32 rows: [q | gate] per query head, then k, then v; engine/kernels_qwen35.js:36-38), the WGSL attnPrep
// (:18-69) done here: q and the new key normalised with (1 + w) and rotated at the token's position pos =
// cache_len[b]; the cache holds keys 0 .. pos - 1, and split 0's block appends the new key and value to the caches
// at pos (when pos < max_len) and folds the token's own key into its partial. No block of the launch reads cache
// row pos for a key it uses (a block's keys end below pos; rows past a span are loaded from clamped rows and masked),
// so the append needs no ordering against the other blocks.
struct DecQ {
  const void* q;
  int64_t ldy;       // FP: row stride of y (floats)
  const float* qnw;  // FP: q_norm weight [D]
  const float* knw;  // FP: k_norm weight [D]
  float eps;
  __bf16* kw;        // FP: the caches, for the append
  __bf16* vw;
};

template <int G, int NT, bool FP>
__global__ __launch_bounds__(256) void attn_decode_partial_kernel(
    DecQ dq, const __bf16* __restrict__ kc, const __bf16* __restrict__ vc,
    const int32_t* __restrict__ cache_len, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int rot,
    float* __restrict__ part, int Hq, int Hkv, int max_len, int S, float scale) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8, "heads per kv head");
  constexpr int NG = (G + 3) / 4;  // lane groups of the MFMA D tile that hold real heads
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  Q35_ARGS_UPFRONT(dq.q, dq.ldy, dq.qnw, dq.knw, dq.eps, dq.kw, dq.vw, kc, vc, cache_len, cos_t, sin_t, rot, part, Hq,
                   Hkv, max_len, S, scale);

  // cache_len lives on the device: its read is issued here and waited for after the query loads below
  const int len_raw = cache_len[b];
  // 0. the raw query loads go out next: they do not depend on the cache length, whose read from device memory
  // is a round trip of its own. Thread t takes quads of 4 dims (qi = t, t + 256, ...), with the rotation partner
  // of each rotary quad; every load is unconditional (clamped indices, results selected afterwards). A wave's 64
  // quads are one head's 256 dims (G * 64 quads over 256 threads), so its RMS is one wave sum.
  const int half = rot >> 1;
  constexpr int NQ = (G * 64 + 255) / 256;
  u32x2 xq[NQ], pq[NQ];
  f32x4 xf[NQ], pf[NQ], wx[NQ], wp[NQ];
  // FP, split 0: the new token's key quad (wave 0: dims 4 lane .., with its rotation partner) and value quad (wave 1)
  const bool newkey = FP && s == 0;
  f32x4 nx, npx, nw, npw;
  if constexpr (FP) {
    const float* yr = static_cast<const float*>(dq.q) + (size_t)b * dq.ldy;
    const float* yb = yr + (size_t)kvh * G * 2 * kDecD;
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int qi = min(tid + 256 * u, G * 64 - 1), hh = qi >> 6, d0 = 4 * (qi & 63);
      const int pd0 = d0 < rot ? (d0 < half ? d0 + half : d0 - half) : d0;
      xf[u] = *reinterpret_cast<const f32x4*>(yb + hh * 2 * kDecD + d0);
      pf[u] = *reinterpret_cast<const f32x4*>(yb + hh * 2 * kDecD + pd0);
      wx[u] = *reinterpret_cast<const f32x4*>(dq.qnw + d0);
      wp[u] = *reinterpret_cast<const f32x4*>(dq.qnw + pd0);
    }
    if (newkey && wave < 2) {
      const int d0 = 4 * lane, pd0 = d0 < rot ? (d0 < half ? d0 + half : d0 - half) : d0;
      const float* src = yr + (size_t)Hq * 2 * kDecD + (size_t)(wave == 0 ? kvh : Hkv + kvh) * kDecD;
      nx = *reinterpret_cast<const f32x4*>(src + d0);
      if (wave == 0) {
        npx = *reinterpret_cast<const f32x4*>(src + pd0);
        nw = *reinterpret_cast<const f32x4*>(dq.knw + d0);
        npw = *reinterpret_cast<const f32x4*>(dq.knw + pd0);
      }
    }
  } else {
    const __bf16* qb = static_cast<const __bf16*>(dq.q) + ((size_t)b * Hq + (size_t)kvh * G) * kDecD;
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int qi = min(tid + 256 * u, G * 64 - 1), hh = qi >> 6, d0 = 4 * (qi & 63);
      const int pd0 = d0 < rot ? (d0 < half ? d0 + half : d0 - half) : d0;
      xq[u] = *reinterpret_cast<const u32x2*>(qb + hh * kDecD + d0);
      pq[u] = *reinterpret_cast<const u32x2*>(qb + hh * kDecD + pd0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // the cache length (FP: the position) is clamped rather than trusted: 0 <= len <= max_len
  const int len = min(max(len_raw, 0), max_len);
  constexpr int L = 4 * kDecTile * NT;  // keys of the block's span: NT tiles per wave
  const int k_begin = s * L;
  const int k_end = min(k_begin + L, len);
  const int pos = FP ? min(len, max_len - 1) : max(len - 1, 0);  // the query's position

  __shared__ __attribute__((aligned(16))) float qf[G][kDecD];
  __shared__ __attribute__((aligned(16))) float knew[FP ? kDecD : 1], vnew[FP ? kDecD : 1];
  __shared__ float snew[FP ? G : 1];
  __shared__ float pl[4][kDecTile][G];
  __shared__ float comb_o[4][G][kDecD];
  __shared__ float comb_ml[4][G][2];

  // Online-softmax state and the per-tile helpers (qfrag, the query A operand in LDS, is filled in step 2 below;
  // it is read per tile rather than held in registers, which keeps two tiles' K and V in flight within budget)
  __shared__ bf16x8 qfrag[8][64];
  const size_t kvbase = ((size_t)b * Hkv + kvh) * (size_t)max_len * kDecD;
  const __bf16* kb = kc + kvbase;
  const __bf16* vb = vc + kvbase;
  float m_run[4], l_run[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) { m_run[r] = -INFINITY; l_run[r] = 0.f; }
  float acc[G][8];
#pragma unroll
  for (int hh = 0; hh < G; ++hh)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[hh][e] = 0.f;

  const int kn = lane & 15, kg = lane >> 4;  // score-tile coordinates: key column, lane group
  const int d0 = 8 * (lane & 31), kp = lane >> 5;  // PV coordinates: 8 dims, key parity
  // K and V of one 16-key tile: keys past the span are loaded from a clamped row and masked (no branch)
  auto tile_load = [&](int key0, bf16x8 (&kv8)[8], u32x4 (&vraw)[kDecTile / 2]) {
    const int key = key0 + kn;
    const __bf16* krow = kb + (size_t)(key < k_end ? key : min(k_begin, max_len - 1)) * kDecD + 8 * kg;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) kv8[ks] = *reinterpret_cast<const bf16x8*>(krow + 32 * ks);
    // keys past the span read the span's last row: their p is exactly 0, so the finite values they bring add
    // nothing (no select on the loaded data, which would make the load's consumer wait for it here)
#pragma unroll
    for (int i = 0; i < kDecTile / 2; ++i) {
      const int vkey = key0 + 2 * i + kp;
      vraw[i] = *reinterpret_cast<const u32x4*>(vb + (size_t)max(min(vkey, k_end - 1), 0) * kDecD + d0);
    }
  };
  auto tile_compute = [&](int key0, const bf16x8 (&kv8)[8], const u32x4 (&vraw)[kDecTile / 2]) {
    const bool kvalid = key0 + kn < k_end;
    // scores S[head][key] for 16 keys
    f32x4 sc = zero4();
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) sc = mfma16(qfrag[ks][lane], kv8[ks], sc);
    // lane group kg holds heads 4 kg + r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float x = kvalid ? sc[r] * scale : -INFINITY;
      const float mn = fmaxf(m_run[r], row16_max(x));
      const float corr = __expf(m_run[r] - mn);
      const float p = __expf(x - mn);
      l_run[r] = l_run[r] * corr + row16_sum(p);
      m_run[r] = mn;
      if (kg < NG && 4 * kg + r < G) pl[wave][kn][4 * kg + r] = p;
      sc[r] = corr;  // broadcast source for the accumulator rescale below
    }
    __builtin_amdgcn_wave_barrier();
    float corr_h[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
      corr_h[hh] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc[hh & 3]), 16 * (hh >> 2)));
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[hh][e] *= corr_h[hh];
    // P.V: lane takes keys key0 + 2 i + kp (masked keys carry p = 0)
#pragma unroll
    for (int i = 0; i < kDecTile / 2; ++i) {
      const int n = 2 * i + kp;
      const u32x4 raw = vraw[i];
      const float vv[8] = {bf16lo(raw[0]), bf16hi(raw[0]), bf16lo(raw[1]), bf16hi(raw[1]),
                           bf16lo(raw[2]), bf16hi(raw[2]), bf16lo(raw[3]), bf16hi(raw[3])};
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        const float ph = pl[wave][n][hh];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[hh][e] += ph * vv[e];
      }
    }
    __builtin_amdgcn_wave_barrier();
  };
  // 1. the G query heads of this kv head, rotated at position pos, in fp32: the cos / sin rows of pos (all loads
  // issued together). rot is a multiple of 8, so no quad straddles rot or rot / 2.
  f32x4 cq[NQ], sq[NQ];
  if (rot > 0) {
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int qi = min(tid + 256 * u, G * 64 - 1), d0 = 4 * (qi & 63);
      const int j0 = d0 < rot ? (d0 < half ? d0 : d0 - half) : 0;
      cq[u] = *reinterpret_cast<const f32x4*>(cos_t + (size_t)pos * half + j0);
      sq[u] = *reinterpret_cast<const f32x4*>(sin_t + (size_t)pos * half + j0);
    }
  }
  // K / V tile registers, two sets used alternately (indices are compile-time after unrolling). Loads are issued
  // for every tile of the span, with rows clamped into the cache, so that none sits behind a branch. The first
  // tile's loads go out right behind the query's (which are older in the queue and return first), so that they
  // travel while the query is rotated and laid out.
  const int key_w = k_begin + kDecTile * wave;
  bf16x8 kt[2][8];
  u32x4 vt[2][kDecTile / 2];
  tile_load(key_w, kt[0], vt[0]);
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int qi = tid + 256 * u, hh = qi >> 6, d0 = 4 * (qi & 63);
    f32x4 x, y;
    if constexpr (FP) {
      // q RMSNorm with (1 + w) (engine/kernels_qwen35.js:40-47); every lane takes part in the wave sum
      const float ss = wave_sum(xf[u][0] * xf[u][0] + xf[u][1] * xf[u][1] + xf[u][2] * xf[u][2] + xf[u][3] * xf[u][3]);
      const float rr = rsqrtf(ss * (1.f / kDecD) + dq.eps);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = xf[u][e] * rr * (1.f + wx[u][e]);
        y[e] = pf[u][e] * rr * (1.f + wp[u][e]);
      }
    } else {
      x = unpack_bf16x4(xq[u]);
      y = unpack_bf16x4(pq[u]);
    }
    if (qi < G * 64) {
      f32x4 r;
      if (d0 < rot) {
        const float sg = d0 < half ? -1.f : 1.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = x[e] * cq[u][e] + sg * y[e] * sq[u][e];
      } else {
        r = x;
      }
      *reinterpret_cast<f32x4*>(&qf[hh][d0]) = r;
    }
  }
  if constexpr (FP) {
    // the new key (split 0, wave 0), normalised and rotated exactly as the front end does it (frontend.hip
    // attn_prep_kernel) and rounded to bf16 as the cache holds it; the value (wave 1) likewise. Lane l holds dims
    // 4 l .. 4 l + 3, whose cos / sin rows wave 0 loaded for its query quad above.
    if (newkey && wave < 2) {
      const int e0 = 4 * lane;
      bf16x4 kb;
      if (wave == 0) {
        const float ss = wave_sum(nx[0] * nx[0] + nx[1] * nx[1] + nx[2] * nx[2] + nx[3] * nx[3]);
        const float rr = rsqrtf(ss * (1.f / kDecD) + dq.eps);
        f32x4 kn, pn, kr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kn[e] = nx[e] * rr * (1.f + nw[e]);
          pn[e] = npx[e] * rr * (1.f + npw[e]);
        }
        if (e0 < rot) {
          const float sg = e0 < half ? -1.f : 1.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) kr[e] = kn[e] * cq[0][e] + sg * pn[e] * sq[0][e];
        } else {
          kr = kn;
        }
        kb = {(__bf16)kr[0], (__bf16)kr[1], (__bf16)kr[2], (__bf16)kr[3]};
      } else {
        kb = {(__bf16)nx[0], (__bf16)nx[1], (__bf16)nx[2], (__bf16)nx[3]};
      }
      float* dst = wave == 0 ? knew : vnew;
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e0 + e] = (float)kb[e];
      if (len < max_len) {
        __bf16* cache = wave == 0 ? dq.kw : dq.vw;
        *reinterpret_cast<bf16x4*>(cache + (((size_t)b * Hkv + kvh) * max_len + len) * kDecD + e0) = kb;
      }
    }
  }
  __syncthreads();

  // 2. A operand: row = head (l % 16 < G), k = dims 32 ks + 8 (l / 16) + j; wave w writes k steps 2 w, 2 w + 1
  {
    const int hr = lane & 15, kgq = lane >> 4;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ks = 2 * wave + u;
      bf16x8 a;
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = (__bf16)(hr < G ? qf[hr][32 * ks + 8 * kgq + j] : 0.f);
      qfrag[ks][lane] = a;
    }
  }
  __syncthreads();


  // 3. tiles key_w + 64 t, t < NT, fully unrolled: tile t + 1's loads are issued before tile t is computed. A
  // tile wholly past the span is loaded (clamped rows) but not computed: its keys carry no weight, and the rows it
  // read may lie beyond the cached length.
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t + 1 < NT) tile_load(key_w + 4 * kDecTile * (t + 1), kt[(t + 1) & 1], vt[(t + 1) & 1]);
    if (key_w + 4 * kDecTile * t < k_end) tile_compute(key_w + 4 * kDecTile * t, kt[t & 1], vt[t & 1]);
  }

  // 4. fold the two key-parity halves, then merge the four waves in LDS
#pragma unroll
  for (int hh = 0; hh < G; ++hh)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[hh][e] += __shfl_xor(acc[hh][e], 32, 64);
  if (lane < 32) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
      for (int e = 0; e < 8; ++e) comb_o[wave][hh][d0 + e] = acc[hh][e];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * kg + r;
    if (kn == 0 && kg < NG && hh < G) {
      comb_ml[wave][hh][0] = m_run[r];
      comb_ml[wave][hh][1] = l_run[r];
    }
  }
  if constexpr (FP) {
    // split 0: the new key's score for each head, from the query and key as the MFMA and the cache hold them (bf16)
    if (newkey) {
      for (int hh = wave; hh < G; hh += 4) {
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) dot += (float)(__bf16)qf[hh][4 * lane + e] * knew[4 * lane + e];
        dot = wave_sum(dot);
        if (lane == 0) snew[hh] = dot * scale;
      }
    }
  }
  __syncthreads();
  float* pb = part + (((size_t)b * Hkv + kvh) * S + s) * (size_t)G * (kDecD + 2);
  for (int i = tid; i < G * kDecD; i += 256) {
    const int hh = i / kDecD, d = i % kDecD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, comb_ml[w][hh][0]);
    float sn = -INFINITY;
    if constexpr (FP) {
      if (newkey) sn = snew[hh];
    }
    M = fmaxf(M, sn);
    float Lsum = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = __expf(comb_ml[w][hh][0] - M);
        Lsum += comb_ml[w][hh][1] * f;
        O += comb_o[w][hh][d] * f;
      }
    }
    if constexpr (FP) {
      if (newkey) {
        const float f = __expf(sn - M);
        Lsum += f;
        O += f * vnew[d];
      }
    }
    pb[(size_t)hh * (kDecD + 2) + d] = O;
    if (d == 0) {
      pb[(size_t)hh * (kDecD + 2) + kDecD] = M;
      pb[(size_t)hh * (kDecD + 2) + kDecD + 1] = Lsum;
    }
  }
}

// Merge over splits, gate, store. One block per (query head, row, slice of 32 head dims): thread (g, d) folds the
// splits g, g + 8, ... of dim d with an online log-sum-exp, loading eight splits' (max, sum, acc) at a time before
// using any of them; the eight groups are combined in LDS.
template <typename Tout, typename Tg>
__global__ __launch_bounds__(256) void attn_decode_merge_kernel(const float* __restrict__ part,
                                                                const Tg* __restrict__ gate, int64_t gate_ld,
                                                                int gate_hs, Tout* __restrict__ out, int Hq, int Hkv,
                                                                int S) {
  Q35_ARGS_UPFRONT(part, gate, gate_ld, gate_hs, out, Hq, Hkv, S);
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int G = Hq / Hkv, kvh = h / G, hh = h % G;
  const int grp = tid >> 5, d = 32 * blockIdx.z + (tid & 31);
  const size_t sstride = (size_t)G * (kDecD + 2);
  const float* pb = part + ((size_t)b * Hkv + kvh) * S * sstride + (size_t)hh * (kDecD + 2);
  __shared__ float gm[8], gl[8], go[8][32];
  // the gate value this thread's output needs is loaded first, so that its round trip overlaps the partials'
  const size_t oi = (size_t)b * Hq * kDecD + (size_t)h * kDecD + d;
  const float gv = tid < 32 ? to_f32(gate[(size_t)b * gate_ld + (size_t)h * gate_hs + d]) : 0.f;
  float M = -INFINITY, Lsum = 0.f, O = 0.f;
  for (int s0 = grp; s0 < S; s0 += 64) {
    float m[8], l[8], a[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int s = min(s0 + 8 * u, S - 1);
      m[u] = pb[(size_t)s * sstride + kDecD];
      l[u] = pb[(size_t)s * sstride + kDecD + 1];
      a[u] = pb[(size_t)s * sstride + d];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (s0 + 8 * u >= S || m[u] == -INFINITY) continue;
      const float mn = fmaxf(M, m[u]);
      const float c0 = __expf(M - mn), c1 = __expf(m[u] - mn);
      Lsum = Lsum * c0 + l[u] * c1;
      O = O * c0 + a[u] * c1;
      M = mn;
    }
  }
  if ((tid & 31) == 0) {
    gm[grp] = M;
    gl[grp] = Lsum;
  }
  go[grp][tid & 31] = O;
  __syncthreads();
  if (tid < 32) {
    float Mx = -INFINITY;
#pragma unroll
    for (int g = 0; g < 8; ++g) Mx = fmaxf(Mx, gm[g]);
    float Lt = 0.f, Ot = 0.f;
    if (Mx != -INFINITY) {
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const float w = gm[g] == -INFINITY ? 0.f : __expf(gm[g] - Mx);
        Lt += gl[g] * w;
        Ot += go[g][tid] * w;
      }
    }
    const float res = Lt > 0.f ? Ot / Lt : 0.f;
    out[oi] = from_f32<Tout>(res * sigmoidf_(gv));
  }
}

// Split of the context: a block's span is 64 NT keys (NT 16-key tiles per wave), NT a power of two <= 16. By
// default the spans are sized so that about 256 blocks (one per CU) cover B x Hkv contexts, with at least one tile
// per wave. Measured over an 8192-key context at B 3 (6 contexts), op time against the span: 1024 keys (8 splits)
// 33.8 us, 512 keys 22.6, 256 keys (32 splits, 192 blocks) 17.8, 128 keys 19.3; spans of 3 and 6 tiles per wave,
// built for the comparison, took 21.7 us (192 keys: 258 blocks, a few CUs take two) and 20.2 us (384 keys). At B 32
// (64 contexts) 4, 8 and 16 splits are within 3 % of each other.
constexpr int kNTs[] = {1, 2, 4, 8, 16};
static int decode_splits(int64_t B, int64_t Hkv, int64_t max_len, int64_t splits, int* nt_out) {
  int64_t S = splits;
  if (S <= 0) {
    const int64_t target = 256;
    S = (target + B * Hkv - 1) / (B * Hkv);
  }
  if (S < 1) S = 1;
  const int64_t L0 = (max_len + S - 1) / S;
  int nt = 16;
  for (int c : kNTs)
    if ((int64_t)64 * c >= L0) {
      nt = c;
      break;
    }
  *nt_out = nt;
  return (int)((max_len + 64 * nt - 1) / (64 * nt));
}

}  // namespace q35

extern "C" size_t q35_gated_attn_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                                        int64_t max_len, int64_t splits) {
  using namespace q35;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_len <= 0) return 0;
  int nt;
  const int S = decode_splits(B, Hkv, max_len, splits, &nt);
  return (size_t)B * Hq * S * (size_t)(D + 2) * sizeof(float);
}

namespace q35 {
// Argument checks shared by both decode entry points (no HIP call).
static int decode_check(const void* q, const void* k_cache, const void* v_cache, const void* gate,
                        const int32_t* cache_len, const float* cos, const float* sin, const void* out, int out_dtype,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, int64_t rot, int64_t splits) {
  if (!q || !k_cache || !v_cache || !gate || !cache_len || !out) return Q35_EINVAL;
  if (out_dtype != Q35_BF16 && out_dtype != Q35_F32) return Q35_EUNSUPPORTED;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_len <= 0 || Hq % Hkv != 0 || rot < 0 || rot > D || (rot & 1))
    return Q35_EINVAL;
  if (rot % 8 != 0) return Q35_EUNSUPPORTED;
  if (rot > 0 && (!cos || !sin)) return Q35_EINVAL;
  if (D != kDecD || B > 65535 || Hkv > 65535) return Q35_EUNSUPPORTED;
  const int64_t G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return Q35_EUNSUPPORTED;
  int nt;
  const int S = decode_splits(B, Hkv, max_len, splits, &nt);
  if ((int64_t)S * 64 * nt > ((int64_t)1 << 31)) return Q35_EUNSUPPORTED;
  return Q35_OK;
}
}  // namespace q35

namespace q35 {
// The two launches of a decode call (partial over the splits, then the merge). FP: the query, the new key and value
// and the gate come from the fused projection output (DecQ), cache_len holding the token's position.
template <bool FP>
static int decode_launch(const DecQ& dq, const void* k_cache, const void* v_cache, const void* gate, int64_t gate_ld,
                         int gate_hs, const int32_t* cache_len, const float* cos, const float* sin, void* out,
                         int out_dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t rot,
                         float scale, int64_t splits, void* workspace, hipStream_t st) {
  const int64_t G = Hq / Hkv;
  int nt;
  const int S = decode_splits(B, Hkv, max_len, splits, &nt);
  float* part = (float*)workspace;
  dim3 grid(S, (unsigned)Hkv, (unsigned)B), block(256);
#define Q35_DEC_LAUNCH(GG, NT)                                                                                   \
  hipLaunchKernelGGL((attn_decode_partial_kernel<GG, NT, FP>), grid, block, 0, st, dq, (const __bf16*)k_cache,  \
                     (const __bf16*)v_cache, cache_len, cos, sin, (int)rot, part, (int)Hq, (int)Hkv,             \
                     (int)max_len, S, scale)
#define Q35_DEC_NT(GG)                        \
  switch (nt) {                               \
    case 1: Q35_DEC_LAUNCH(GG, 1); break;     \
    case 2: Q35_DEC_LAUNCH(GG, 2); break;     \
    case 4: Q35_DEC_LAUNCH(GG, 4); break;     \
    case 8: Q35_DEC_LAUNCH(GG, 8); break;     \
    default: Q35_DEC_LAUNCH(GG, 16); break;   \
  }
  switch (G) {
    case 1: Q35_DEC_NT(1); break;
    case 2: Q35_DEC_NT(2); break;
    case 4: Q35_DEC_NT(4); break;
    default: Q35_DEC_NT(8); break;
  }
#undef Q35_DEC_NT
#undef Q35_DEC_LAUNCH
  using Tg = typename std::conditional<FP, float, __bf16>::type;
  const dim3 mgrid((unsigned)Hq, (unsigned)B, kDecD / 32);
  if (out_dtype == Q35_F32)
    hipLaunchKernelGGL((attn_decode_merge_kernel<float, Tg>), mgrid, dim3(256), 0, st, part, (const Tg*)gate, gate_ld,
                       gate_hs, (float*)out, (int)Hq, (int)Hkv, S);
  else
    hipLaunchKernelGGL((attn_decode_merge_kernel<__bf16, Tg>), mgrid, dim3(256), 0, st, part, (const Tg*)gate,
                       gate_ld, gate_hs, (__bf16*)out, (int)Hq, (int)Hkv, S);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
}  // namespace q35

extern "C" int q35_gated_attn_decode(const void* q, const void* k_cache, const void* v_cache, const void* gate,
                                     const int32_t* cache_len, const float* cos, const float* sin, void* out,
                                     int out_dtype,
                                     int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, int64_t rot,
                                     float scale, int64_t splits, void* workspace, size_t workspace_bytes,
                                     q35_stream_t stream) {
  using namespace q35;
  const int chk = decode_check(q, k_cache, v_cache, gate, cache_len, cos, sin, out, out_dtype, B, Hq, Hkv, D,
                               max_len, rot, splits);
  if (chk != Q35_OK) return chk;
  const size_t need = q35_gated_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, splits);
  if (!workspace || workspace_bytes < need) return Q35_EWORKSPACE;
  const DecQ dq{q, 0, nullptr, nullptr, 0.f, nullptr, nullptr};
  return decode_launch<false>(dq, k_cache, v_cache, gate, Hq * D, (int)D, cache_len, cos, sin, out, out_dtype, B,
                              Hq, Hkv, max_len, rot, scale, splits, workspace, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int q35_gated_attn_decode_proj(const float* y, int64_t ldy, const float* q_norm_w, const float* k_norm_w,
                                          float eps, void* k_cache, void* v_cache, const int32_t* pos,
                                          const float* cos, const float* sin, void* out, int out_dtype, int64_t B,
                                          int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, int64_t rot,
                                          float scale, int64_t splits, void* workspace, size_t workspace_bytes,
                                          q35_stream_t stream) {
  using namespace q35;
  if (!y || !q_norm_w || !k_norm_w) return Q35_EINVAL;
  const int chk = decode_check(y, k_cache, v_cache, y, pos, cos, sin, out, out_dtype, B, Hq, Hkv, D, max_len, rot,
                               splits);
  if (chk != Q35_OK) return chk;
  if (ldy < Hq * 2 * D + 2 * Hkv * D) return Q35_EINVAL;
  // y, its rows and the norm weights are read as 16-byte vectors
  if ((ldy & 3) || ((uintptr_t)y & 15) || ((uintptr_t)q_norm_w & 15) || ((uintptr_t)k_norm_w & 15))
    return Q35_EUNSUPPORTED;
  if (B * ldy > ((int64_t)1 << 40)) return Q35_EUNSUPPORTED;
  const size_t need = q35_gated_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, splits);
  if (!workspace || workspace_bytes < need) return Q35_EWORKSPACE;
  const DecQ dq{y, ldy, q_norm_w, k_norm_w, eps, (__bf16*)k_cache, (__bf16*)v_cache};
  // the gate of head h: columns h 2 D + D .. of y
  return decode_launch<true>(dq, k_cache, v_cache, y + D, ldy, (int)(2 * D), pos, cos, sin, out, out_dtype, B, Hq,
                             Hkv, max_len, rot, scale, splits, workspace, reinterpret_cast<hipStream_t>(stream));
}

// ---- Allocation-free variant. The split-K partials live in a fixed device array of this file instead of a caller
// workspace. Each device holds its own copy of the array (for the life of the process); its address on a device is
// resolved once, on the first call with that device current, and kept per device. Every call on a device shares the
// array: calls that overlap on one device race. Nothing in it needs clearing between calls: every partial the merge
// reads is written by the same call's first kernel (an empty split writes max -inf, sum 0).
namespace q35 {
constexpr size_t kNoAllocScratchBytes = (size_t)9 << 20;
constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;
}  // namespace q35

static __device__ __align__(256) unsigned char scratch[q35::kNoAllocScratchBytes];

namespace q35 {
// The device address of `scratch` on the current device (the host-side name is only a stand-in for the symbol).
static int scratch_on_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return Q35_ELAUNCH;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return Q35_ELAUNCH;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return Q35_OK;
}
}  // namespace q35

extern "C" size_t q35_gated_attn_decode_noalloc_max_bytes(void) { return q35::kNoAllocScratchBytes; }

extern "C" int q35_gated_attn_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                             const void* gate, const int32_t* cache_len, const float* cos,
                                             const float* sin, void* out, int out_dtype, int64_t B, int64_t Hq,
                                             int64_t Hkv, int64_t D, int64_t max_len, int64_t rot, float scale,
                                             int64_t splits, q35_stream_t stream) {
  using namespace q35;
  const int chk = decode_check(q, k_cache, v_cache, gate, cache_len, cos, sin, out, out_dtype, B, Hq, Hkv, D,
                               max_len, rot, splits);
  if (chk != Q35_OK) return chk;
  if (q35_gated_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, splits) > kNoAllocScratchBytes)
    return Q35_ESCRATCH;
  void* ws = nullptr;
  const int st = scratch_on_current_device(&ws);
  if (st != Q35_OK) return st;
  return q35_gated_attn_decode(q, k_cache, v_cache, gate, cache_len, cos, sin, out, out_dtype, B, Hq, Hkv, D,
                               max_len, rot, scale, splits, ws, kNoAllocScratchBytes, stream);
}
