// Gated causal GQA attention prefill with partial RoPE and the sigmoid output gate fused (flash-style, MFMA bf16).
//
// Semantics (HF:656-698, eager_attention_forward HF:604-626, apply_rotary_pos_emb HF:554-589; WGSL
// engine/kernels_qwen35.js:50-59 and :73-123):
//   q, k  <- partial RoPE on dims [0, rot): x * cos + rotate_half(x) * sin, pairs (i, i + rot/2), position pos0 + t
//   o_h    = softmax(q_h K^T * scale + causal mask) V     (fp32 softmax; kv head h / (Hq / Hkv))
//   out    = o * sigmoid(gate)
//
// Decomposition: one block per (32-query block, group of up to 4 query heads sharing a kv head, batch row); wave w
// of the block owns query head w of the group, so every K/V tile staged in LDS serves up to 4 heads. Query blocks
// are issued longest (latest) first to shorten the causal tail.
// Per 32-key tile each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (K from LDS, Q^T resident in
// registers as the B operand), so a query's 16 scores sit in one lane (row max / sum need one cross-half exchange),
// then O^T += V^T P^T where P^T's accumulator layout is used directly as the B operand (k permutation of the keys;
// the V^T operand in LDS is read with the same permutation). K tiles are rotated while staged; V tiles are
// transposed while staged (4 keys x 8 dims per thread). Two LDS stages, one barrier per tile.
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kPD = 256;            // head dim
constexpr int kBQ = 32;             // queries per wave
constexpr int kBK = 32;             // keys per tile
constexpr int kKS = kPD + 8;        // K tile row stride (elements): 528 B, conflict-free 16-byte reads
constexpr int kVS = kBK + 4;        // V^T row stride (elements): 72 B, conflict-free 8-byte reads
constexpr int kRotMax = 64;         // rotary dims supported by the fused rotation (Qwen3.5: 64)
constexpr int kHM = kRotMax / 2;    // cos / sin entries per position

template <int GW>
__global__ __launch_bounds__(64 * GW) void attn_prefill_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    const __bf16* __restrict__ gate, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int pos0,
    __bf16* __restrict__ out, int T, int Hq, int Hkv, int ngroups, int rot, float scale, int nqb, int B) {
  constexpr int NT = 64 * GW;
  __shared__ __attribute__((aligned(16))) __bf16 ks_lds[2][kBK * kKS];
  __shared__ __attribute__((aligned(16))) __bf16 vt_lds[2][kPD * kVS];
  __shared__ __attribute__((aligned(16))) float rope_lds[2][kBK][2 * kHM];  // cos | sin of the staged tile's keys

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_other = B * Hkv * ngroups;
  const int qb = nqb - 1 - (int)(blockIdx.x / n_other);
  const int rem = blockIdx.x % n_other;
  const int b = rem / (Hkv * ngroups);
  const int kvh = (rem / ngroups) % Hkv;
  const int hg = rem % ngroups;
  const int G = Hq / Hkv;
  const int h = kvh * G + hg * GW + wave;
  const int q0 = qb * kBQ;
  const int half = rot >> 1;

  const int ln = lane & 31, hh = lane >> 5;

  // ---- Q^T operand (B of S^T = K Q^T): lane holds query q0 + ln, dims 16 ks + 8 hh + j ----
  bf16x8 qop[16];
  {
    const int t = q0 + ln;
    const bool tv = t < T;
    const __bf16* qrow = q + (((size_t)b * T + (tv ? t : 0)) * Hq + h) * kPD;
    const int pos = pos0 + t;
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      const int d = 16 * ks + 8 * hh;
      const uint4 raw = *reinterpret_cast<const uint4*>(qrow + d);
      float x[8] = {bf16lo(raw.x), bf16hi(raw.x), bf16lo(raw.y), bf16hi(raw.y),
                    bf16lo(raw.z), bf16hi(raw.z), bf16lo(raw.w), bf16hi(raw.w)};
      if (tv && d < rot) {
        const int pd = d < half ? d + half : d - half;
        const uint4 pr = *reinterpret_cast<const uint4*>(qrow + pd);
        const float y[8] = {bf16lo(pr.x), bf16hi(pr.x), bf16lo(pr.y), bf16hi(pr.y),
                            bf16lo(pr.z), bf16hi(pr.z), bf16lo(pr.w), bf16hi(pr.w)};
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

  // ---- staging of one K/V tile: global -> registers -> (rotate / transpose) -> LDS ----
  // K chunks are numbered rotary chunks first (32 rows x RC chunks of 8 dims, RC = rot / 8), then the rest, so the
  // rotary work spreads over the threads. The cos/sin rows of the tile's 32 keys are loaded with the tile and
  // passed through LDS (one float4 of the table slice per thread per array).
  constexpr int KCH = kBK * (kPD / 8) / NT;  // 16-byte K chunks per thread
  constexpr int VUN = (kBK / 4) * (kPD / 8) / NT;  // (4 keys x 8 dims) V units per thread
  constexpr int RQ = (kBK * kHM / 4 + NT - 1) / NT;  // float4s of each rope table slice per thread
  const int RC = rot / 8;
  // rotary chunks come first, so with rot <= 64 only the first KPAR chunks of a thread can need a partner chunk
  constexpr int KPAR = (kBK * (kRotMax / 8) + NT - 1) / NT;
  u32x4 kreg[KCH], kpar[KPAR], vreg[VUN][4];
  f32x4 creg[RQ > 0 ? RQ : 1], sreg[RQ > 0 ? RQ : 1];
  const __bf16* kbase = k + ((size_t)b * T * Hkv + kvh) * kPD;  // + (key * Hkv) * kPD
  const __bf16* vbase = v + ((size_t)b * T * Hkv + kvh) * kPD;
  auto kchunk = [&](int c, int& row, int& cc) {
    if (c < kBK * RC) {
      row = c / RC;
      cc = c % RC;
    } else {
      const int c2 = c - kBK * RC;
      row = c2 / (32 - RC);
      cc = RC + c2 % (32 - RC);
    }
  };
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      int row, cc;
      kchunk(tid + i * NT, row, cc);
      // loads are unconditional from clamped rows (a load whose use sits in a branch is waited for in place);
      // rows past T are zeroed when the tile is written to LDS
      const int key = min(kt * kBK + row, T - 1);
      const __bf16* kr = kbase + (size_t)key * Hkv * kPD;
      kreg[i] = *reinterpret_cast<const u32x4*>(kr + 8 * cc);
      if (i < KPAR) {
        const int pd = cc < RC ? (8 * cc < half ? 8 * cc + half : 8 * cc - half) : 8 * cc;
        kpar[i < KPAR ? i : 0] = *reinterpret_cast<const u32x4*>(kr + pd);
      }
    }
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
      // table slice [32 keys][half] of cos and sin, as float4s
      const int e4 = tid + i * NT;  // float4 index within the slice
      const int row = e4 / (kHM / 4), j4 = e4 % (kHM / 4);
      const int key = min(kt * kBK + min(row, kBK - 1), T - 1);
      const int jc = min(4 * j4, half - 4);  // entries past rot/2 are never read back
      creg[i] = *reinterpret_cast<const f32x4*>(cos_t + (size_t)(pos0 + key) * half + jc);
      sreg[i] = *reinterpret_cast<const f32x4*>(sin_t + (size_t)(pos0 + key) * half + jc);
    }
#pragma unroll
    for (int i = 0; i < VUN; ++i) {
      const int u = tid + i * NT, dc = u >> 3, kq = u & 7;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = min(kt * kBK + 4 * kq + r, T - 1);
        vreg[i][r] = *reinterpret_cast<const u32x4*>(vbase + (size_t)key * Hkv * kPD + 8 * dc);
      }
    }
  };
  auto store_tile = [&](int kt, int buf) {
    if (rot > 0) {
      float* rl = &rope_lds[buf][0][0];
#pragma unroll
      for (int i = 0; i < RQ; ++i) {
        const int e4 = tid + i * NT;
        const int row = e4 / (kHM / 4), j4 = e4 % (kHM / 4);
        if (e4 < kBK * kHM / 4) {
          *reinterpret_cast<f32x4*>(rl + row * (2 * kHM) + 4 * j4) = creg[i];
          *reinterpret_cast<f32x4*>(rl + row * (2 * kHM) + kHM + 4 * j4) = sreg[i];
        }
      }
      __syncthreads();
    }
    __bf16* kl = ks_lds[buf];
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      int row, cc;
      kchunk(tid + i * NT, row, cc);
      const u32x4 z = {0u, 0u, 0u, 0u};
      const bool kvalid = kt * kBK + row < T;
      u32x4 w = kvalid ? kreg[i] : z;
      const int d = 8 * cc;
      if (i < KPAR && cc < RC && kvalid) {
        const float* cr = &rope_lds[buf][row][0];
        const float* sr = cr + kHM;
        const int j0 = d < half ? d : d - half;
        const float sg = d < half ? -1.f : 1.f;
        const u32x4 p = kpar[i < KPAR ? i : 0];
        const float x[8] = {bf16lo(w[0]), bf16hi(w[0]), bf16lo(w[1]), bf16hi(w[1]),
                            bf16lo(w[2]), bf16hi(w[2]), bf16lo(w[3]), bf16hi(w[3])};
        const float y[8] = {bf16lo(p[0]), bf16hi(p[0]), bf16lo(p[1]), bf16hi(p[1]),
                            bf16lo(p[2]), bf16hi(p[2]), bf16lo(p[3]), bf16hi(p[3])};
        bf16x8 o8;
#pragma unroll
        for (int j = 0; j < 8; ++j) o8[j] = (__bf16)(x[j] * cr[j0 + j] + sg * y[j] * sr[j0 + j]);
        w = __builtin_bit_cast(u32x4, o8);
      }
      *reinterpret_cast<u32x4*>(kl + row * kKS + 8 * cc) = w;
    }
    __bf16* vl = vt_lds[buf];
#pragma unroll
    for (int i = 0; i < VUN; ++i) {
      const int u = tid + i * NT, dc = u >> 3, kq = u & 7;
      const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int r = 0; r < 4; ++r) vreg[i][r] = kt * kBK + 4 * kq + r < T ? vreg[i][r] : z;
      // transpose 4 keys x 8 dims -> 8 dims x 4 keys (component selects: taking the address of a register array
      // would move it to scratch)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        auto h16 = [&](const u32x4& r) -> uint32_t {
          const uint32_t w = r[e >> 1];
          return (e & 1) ? (w >> 16) : (w & 0xffffu);
        };
        u32x2 pk;
        pk[0] = h16(vreg[i][0]) | (h16(vreg[i][1]) << 16);
        pk[1] = h16(vreg[i][2]) | (h16(vreg[i][3]) << 16);
        *reinterpret_cast<u32x2*>(vl + (8 * dc + e) * kVS + 4 * kq) = pk;
      }
    }
  };

  const int nkt_all = (T + kBK - 1) / kBK;
  const int nkt = min(nkt_all, (q0 + kBQ - 1) / kBK + 1);

  f32x16 o[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o[mt] = zero16();
  float m_run = -INFINITY, l_run = 0.f;
  const int tq = q0 + ln;  // this lane's query

  load_tile(0);
  store_tile(0, 0);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nkt) load_tile(kt + 1);
    // S^T = K Q^T: rows = 32 keys, cols = 32 queries
    const __bf16* kl = ks_lds[buf];
    f32x16 s = zero16(), s2 = zero16();  // two independent chains over the 16 K steps
#pragma unroll
    for (int ks = 0; ks < 16; ks += 2) {
      const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(kl + ln * kKS + 16 * ks + 8 * hh);
      const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(kl + ln * kKS + 16 * (ks + 1) + 8 * hh);
      s = mfma32(a0, qop[ks], s);
      s2 = mfma32(a1, qop[ks + 1], s2);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] += s2[r];
    // online softmax along the keys of this lane's query. The running max is only moved (and O, l rescaled) when
    // a row max exceeds it by more than 8 (natural log units): p = exp(s - m) then stays <= e^8, exact enough in
    // fp32 and in the bf16 P operand, and most tiles skip the 128-register rescale.
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kt * kBK + 8 * (r >> 2) + 4 * hh + (r & 3);
      const float x = (key <= tq && key < T) ? s[r] * scale : -INFINITY;
      s[r] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (__any(mx > m_run + 8.f)) {
      const float mn = fmaxf(m_run, mx);
      const float corr = __expf(m_run - mn);
      l_run *= corr;
      m_run = mn;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mt][r] *= corr;
    }
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __expf(s[r] - m_run);
      ps += s[r];
    }
    ps += __shfl_xor(ps, 32, 64);
    l_run += ps;
    bf16x8 pb[2];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pb[0][j] = (__bf16)s[j];
      pb[1][j] = (__bf16)s[8 + j];
    }
    // O^T += V^T P^T: rows = 256 dims (8 tiles), k = 32 keys (2 steps)
    const __bf16* vl = vt_lds[buf];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const __bf16* vr = vl + (32 * mt + ln) * kVS + 16 * kk + 4 * hh;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vr);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vr + 8);
        const u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
        o[mt] = mfma32(__builtin_bit_cast(bf16x8, w), pb[kk], o[mt]);
      }
    }
    if (kt + 1 < nkt) store_tile(kt + 1, buf ^ 1);
    __syncthreads();
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
        const uint2 gr = *reinterpret_cast<const uint2*>(gate + rowo + d);
        const float gv[4] = {bf16lo(gr.x), bf16hi(gr.x), bf16lo(gr.y), bf16hi(gr.y)};
        bf16x4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (__bf16)(o[mt][4 * c + e] * inv * sigmoidf_(gv[e]));
        *reinterpret_cast<bf16x4*>(out + rowo + d) = ov;
      }
    }
  }
}

}  // namespace q35

extern "C" int q35_gated_attn_prefill(const void* q, const void* k, const void* v, const void* gate,
                                      const float* cos, const float* sin, int64_t pos0, void* out, int64_t B,
                                      int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t rot, float scale,
                                      q35_stream_t stream) {
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
  const int64_t nqb = (T + kBQ - 1) / kBQ;
  const int64_t nblocks = nqb * B * Hkv * ngroups;
  if (nblocks > 0x7fffffff || T * Hq * D > ((int64_t)1 << 40)) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define Q35_PF_LAUNCH(GG)                                                                                      \
  hipLaunchKernelGGL(attn_prefill_kernel<GG>, dim3((unsigned)nblocks), dim3(64 * GG), 0, st, (const __bf16*)q, \
                     (const __bf16*)k, (const __bf16*)v, (const __bf16*)gate, cos, sin, (int)pos0, (__bf16*)out,  \
                     (int)T, (int)Hq, (int)Hkv, ngroups, (int)rot, scale, (int)nqb, (int)B)
  switch (GW) {
    case 1: Q35_PF_LAUNCH(1); break;
    case 2: Q35_PF_LAUNCH(2); break;
    default: Q35_PF_LAUNCH(4); break;
  }
#undef Q35_PF_LAUNCH
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
