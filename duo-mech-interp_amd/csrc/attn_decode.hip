// Gated GQA attention decode: one new query token per row over a bf16 KV cache, split-K over the context.
//
// Semantics (HF:656-698 with a cache, eager_attention_forward HF:604-626; WGSL engine/kernels_qwen35.js:73-123):
//   q_h   <- partial RoPE at position cache_len[b] - 1 (pairs (i, i + rot/2) on the first rot dims, HF:554-589)
//   o_h    = softmax(q_h . K^T * scale) V      over keys 0 .. cache_len[b]-1 of kv head h / (Hq / Hkv)
//   out_h  = o_h * sigmoid(gate_h)             (HF:698)
//
// Pass 1 (attn_decode_partial_kernel): one block of 4 waves per (split, kv head, row). The G = Hq / Hkv query heads
// that share a kv head are the M rows of one 16x16x32 MFMA tile, so each K row is read from HBM once for all G
// heads. Each wave walks 16-key tiles of the block's span: scores via 8 MFMAs whose B operand is loaded straight
// from the cache (16 contiguous bytes per lane), an online softmax on the 16 columns, then P.V on the vector ALU with
// fully coalesced 16-byte V-row loads (32 lanes cover one 512-byte row). The four waves' (max, sum, acc) are merged
// in LDS and written as one partial per (row, kv head, split).
// Pass 2 (attn_decode_merge_kernel): log-sum-exp merge over splits, sigmoid gate, bf16 store.
// HBM traffic is the K and V spans once (AI ~ 4 flop/byte): the kernel is bandwidth bound by design.
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kDecD = 256;  // head dim
constexpr int kDecTile = 16;

template <int G>
__global__ __launch_bounds__(256) void attn_decode_partial_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ kc, const __bf16* __restrict__ vc,
    const int32_t* __restrict__ cache_len, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int rot,
    float* __restrict__ part, int Hq, int Hkv, int max_len, int S, int L, float scale) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8, "heads per kv head");
  constexpr int NG = (G + 3) / 4;  // lane groups of the MFMA D tile that hold real heads
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  // cache_len lives on the device, so it is clamped here rather than trusted: 0 <= len <= max_len
  const int len = min(max(cache_len[b], 0), max_len);
  const int k_begin = s * L;
  const int k_end = min(k_begin + L, len);
  const int pos = max(len - 1, 0);

  __shared__ float qf[G][kDecD];
  __shared__ float pl[4][kDecTile][G];
  __shared__ float comb_o[4][G][kDecD];
  __shared__ float comb_ml[4][G][2];

  // Online-softmax state and the per-tile helpers (qa, the query A operand, is filled in step 2 below)
  bf16x8 qa[8];
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
    const __bf16* krow = kb + (size_t)(key < k_end ? key : k_begin) * kDecD + 8 * kg;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) kv8[ks] = *reinterpret_cast<const bf16x8*>(krow + 32 * ks);
#pragma unroll
    for (int i = 0; i < kDecTile / 2; ++i) {
      const int vkey = key0 + 2 * i + kp;
      const u32x4 z = {0u, 0u, 0u, 0u};
      const u32x4 ld = *reinterpret_cast<const u32x4*>(vb + (size_t)min(vkey, k_end - 1) * kDecD + d0);
      vraw[i] = vkey < k_end ? ld : z;
    }
  };
  auto tile_compute = [&](int key0, const bf16x8 (&kv8)[8], const u32x4 (&vraw)[kDecTile / 2]) {
    const bool kvalid = key0 + kn < k_end;
    // scores S[head][key] for 16 keys
    f32x4 sc = zero4();
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) sc = mfma16(qa[ks], kv8[ks], sc);
    // lane group kg holds heads 4 kg + r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float x = kvalid ? sc[r] * scale : -INFINITY;
      float tm = x;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) tm = fmaxf(tm, __shfl_xor(tm, off, 64));
      const float mn = fmaxf(m_run[r], tm);
      const float corr = __expf(m_run[r] - mn);
      const float p = __expf(x - mn);
      float ps = p;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) ps += __shfl_xor(ps, off, 64);
      l_run[r] = l_run[r] * corr + ps;
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
    // P.V: lane takes keys key0 + 2 i + kp (masked keys were loaded as zeros and carry p = 0)
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
  // first tile pair's K and V loads go out before the q prologue (they do not depend on q)
  int key0 = k_begin + kDecTile * wave;
  bf16x8 ka[8], kb2[8];
  u32x4 va[kDecTile / 2], vb2[kDecTile / 2];
  bool two = key0 + 4 * kDecTile < k_end;
  if (key0 < k_end) {
    tile_load(key0, ka, va);
    if (two) tile_load(key0 + 4 * kDecTile, kb2, vb2);
  }

  // 1. the G query heads of this kv head, rotated at position pos, in fp32 (all loads of a thread issued together)
  {
    const __bf16* qb = q + ((size_t)b * Hq + (size_t)kvh * G) * kDecD;
    const int half = rot >> 1;
    constexpr int NQ = G * kDecD / 256;
    float x[NQ], pr[NQ], c[NQ], sn[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int i = tid + 256 * u, hh = i / kDecD, d = i % kDecD;
      const bool rotd = d < rot;
      const int j = d < half ? d : d - half;
      x[u] = (float)qb[hh * kDecD + d];
      pr[u] = (float)qb[hh * kDecD + (rotd ? (d < half ? d + half : d - half) : d)];
      c[u] = rotd ? cos_t[(size_t)pos * half + j] : 1.f;
      sn[u] = rotd ? sin_t[(size_t)pos * half + j] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int i = tid + 256 * u, hh = i / kDecD, d = i % kDecD;
      qf[hh][d] = d < half ? x[u] * c[u] - pr[u] * sn[u] : x[u] * c[u] + pr[u] * sn[u];
    }
  }
  __syncthreads();

  // 2. A operand: row = head (l % 16 < G), k = dims 32 ks + 8 (l / 16) + j
  {
    const int hr = lane & 15, kgq = lane >> 4;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) qa[ks][j] = (__bf16)(hr < G ? qf[hr][32 * ks + 8 * kgq + j] : 0.f);
  }

  // 3. tiles key0 = k_begin + 16 wave + 64 i, two per iteration: both tiles' loads are in flight before the first
  // tile's math (the second only when the wave has it); the first pair is issued before the q prologue above
  for (; key0 < k_end;) {
    tile_compute(key0, ka, va);
    if (two) tile_compute(key0 + 4 * kDecTile, kb2, vb2);
    key0 += 8 * kDecTile;
    if (key0 < k_end) {
      two = key0 + 4 * kDecTile < k_end;
      tile_load(key0, ka, va);
      if (two) tile_load(key0 + 4 * kDecTile, kb2, vb2);
    }
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
  __syncthreads();
  float* pb = part + (((size_t)b * Hkv + kvh) * S + s) * (size_t)G * (kDecD + 2);
  for (int i = tid; i < G * kDecD; i += 256) {
    const int hh = i / kDecD, d = i % kDecD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, comb_ml[w][hh][0]);
    float Lsum = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = __expf(comb_ml[w][hh][0] - M);
        Lsum += comb_ml[w][hh][1] * f;
        O += comb_o[w][hh][d] * f;
      }
    }
    pb[(size_t)hh * (kDecD + 2) + d] = O;
    if (d == 0) {
      pb[(size_t)hh * (kDecD + 2) + kDecD] = M;
      pb[(size_t)hh * (kDecD + 2) + kDecD + 1] = Lsum;
    }
  }
}

// Merge over splits, gate, store. One block per (query head, row, quarter of the head dims): the split weights
// exp(m_s - M) are formed once in LDS, then four groups of 64 threads each fold a quarter of the splits for one dim
// per thread (256-byte coalesced loads), and the four groups are summed in LDS.
__global__ __launch_bounds__(256) void attn_decode_merge_kernel(const float* __restrict__ part,
                                                                const __bf16* __restrict__ gate,
                                                                __bf16* __restrict__ out, int Hq, int Hkv, int S) {
  const int h = blockIdx.x, b = blockIdx.y, dq = blockIdx.z, tid = threadIdx.x;
  const int G = Hq / Hkv, kvh = h / G, hh = h % G;
  const size_t sstride = (size_t)G * (kDecD + 2);
  const float* pb = part + ((size_t)b * Hkv + kvh) * S * sstride + (size_t)hh * (kDecD + 2);
  extern __shared__ float wsh[];  // [S] weights
  __shared__ float red[2][4];
  __shared__ float accs[4][64];
  // global max over splits
  float mx = -INFINITY;
  for (int s = tid; s < S; s += 256) mx = fmaxf(mx, pb[s * sstride + kDecD]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if ((tid & 63) == 0) red[0][tid >> 6] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  float ls = 0.f;
  for (int s = tid; s < S; s += 256) {
    const float ms = pb[s * sstride + kDecD];
    const float w = (ms == -INFINITY || M == -INFINITY) ? 0.f : __expf(ms - M);
    wsh[s] = w;
    ls += w * pb[s * sstride + kDecD + 1];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ls += __shfl_xor(ls, o, 64);
  if ((tid & 63) == 0) red[1][tid >> 6] = ls;
  __syncthreads();
  const float Lsum = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  const int grp = tid >> 6, d = 64 * dq + (tid & 63);
  float acc = 0.f;
  int s = grp;
  for (; s + 28 < S; s += 32) {  // eight independent loads in flight per thread
    float x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = pb[(size_t)(s + 4 * u) * sstride + d];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += wsh[s + 4 * u] * x[u];
  }
  for (; s < S; s += 4) acc += wsh[s] * pb[(size_t)s * sstride + d];
  accs[grp][tid & 63] = acc;
  __syncthreads();
  if (tid < 64) {
    const float O = accs[0][tid] + accs[1][tid] + accs[2][tid] + accs[3][tid];
    const size_t oi = (size_t)b * Hq * kDecD + (size_t)h * kDecD + d;
    const float res = Lsum > 0.f ? O / Lsum : 0.f;
    out[oi] = (__bf16)(res * sigmoidf_((float)gate[oi]));
  }
}

static int decode_splits(int64_t B, int64_t Hkv, int64_t max_len, int64_t splits, int* L_out) {
  int64_t S = splits;
  if (S <= 0) {
    const int64_t target = 512;  // blocks: two per CU
    S = (target + B * Hkv - 1) / (B * Hkv);
  }
  const int64_t max_s = (max_len + 127) / 128;  // at least two 16-key tiles per wave
  if (S > max_s) S = max_s;
  if (S < 1) S = 1;
  int64_t L = (max_len + S - 1) / S;
  L = (L + 63) / 64 * 64;
  S = (max_len + L - 1) / L;
  *L_out = (int)L;
  return (int)S;
}

}  // namespace q35

extern "C" size_t q35_gated_attn_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                                        int64_t max_len, int64_t splits) {
  using namespace q35;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_len <= 0) return 0;
  int L;
  const int S = decode_splits(B, Hkv, max_len, splits, &L);
  return (size_t)B * Hq * S * (size_t)(D + 2) * sizeof(float);
}

extern "C" int q35_gated_attn_decode(const void* q, const void* k_cache, const void* v_cache, const void* gate,
                                     const int32_t* cache_len, const float* cos, const float* sin, void* out,
                                     int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, int64_t rot,
                                     float scale, int64_t splits, void* workspace, size_t workspace_bytes,
                                     q35_stream_t stream) {
  using namespace q35;
  if (!q || !k_cache || !v_cache || !gate || !cache_len || !out) return Q35_EINVAL;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_len <= 0 || Hq % Hkv != 0 || rot < 0 || rot > D || (rot & 1))
    return Q35_EINVAL;
  if (rot > 0 && (!cos || !sin)) return Q35_EINVAL;
  if (D != kDecD || B > 65535 || Hkv > 65535) return Q35_EUNSUPPORTED;
  const int64_t G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return Q35_EUNSUPPORTED;
  int L;
  const int S = decode_splits(B, Hkv, max_len, splits, &L);
  const size_t need = q35_gated_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, splits);
  if (!workspace || workspace_bytes < need) return Q35_EWORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* part = (float*)workspace;
  dim3 grid(S, (unsigned)Hkv, (unsigned)B), block(256);
#define Q35_DEC_LAUNCH(GG)                                                                                     \
  hipLaunchKernelGGL(attn_decode_partial_kernel<GG>, grid, block, 0, st, (const __bf16*)q,                     \
                     (const __bf16*)k_cache, (const __bf16*)v_cache, cache_len, cos, sin, (int)rot, part, (int)Hq, \
                     (int)Hkv, (int)max_len, S, L, scale)
  switch (G) {
    case 1: Q35_DEC_LAUNCH(1); break;
    case 2: Q35_DEC_LAUNCH(2); break;
    case 4: Q35_DEC_LAUNCH(4); break;
    default: Q35_DEC_LAUNCH(8); break;
  }
#undef Q35_DEC_LAUNCH
  hipLaunchKernelGGL(attn_decode_merge_kernel, dim3((unsigned)Hq, (unsigned)B, kDecD / 64), dim3(256),
                     (size_t)S * sizeof(float), st, part,
                     (const __bf16*)gate, (__bf16*)out, (int)Hq, (int)Hkv, S);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
