// The per-layer work around the two mixers, as HBM-bound passes over the fused projection output y (one GEMM per
// layer produces every projection of a token as one row of y):
//
//   gdn_conv_kernel        (and gdn_conv1_kernel, its T = 1 form) Gated DeltaNet front end (HF:454-499; WGSL conv / convState, engine/kernels_qwen35.js
//                          :127-178, and the gate terms of `delta`, :226-229): causal depthwise conv (K taps, carried
//                          state of the previous K-1 inputs) + SiLU over the q|k|v channels of y, split into dense
//                          q, k [B, T, Hk, dk] and v [B, T, Hv, dv]; beta = sigmoid(b), g = -exp(A_log) *
//                          softplus(a + dt_bias) (softplus threshold 20) from the b and a columns of y; the conv state
//                          advanced by the call's T inputs.
//   gated_rmsnorm_kernel   Qwen3_5RMSNormGated (HF:168-184; engine/kernels_qwen35.js:237-243): per (token, head)
//                          o * rsqrt(mean o^2 + eps) * w * silu(z) * head_scale, with plain w.
//   attn_prep_kernel       attention front end (HF:667-680; WGSL attnPrep, engine/kernels_qwen35.js:18-69): per
//                          head RMSNorm with (1 + w) of q and k, the per-head [q | gate] halves of q_proj split apart,
//                          dense bf16 q, gate, k, v for the prefill kernel, and the rotated keys and the values
//                          written into the bf16 KV cache at positions pos[b] + t (pos read on the device, so that a
//                          captured decode step replays at the right position).
//   add_rmsnorm_kernel     the decoder layer's residual add + RMSNorm with (1 + w) (HF:720-734, :753-793).
#include <type_traits>

#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kConvMaxK = 8;
constexpr int kConvCh = 64;    // channels per conv block (16 quads)
constexpr int kConvTl = 16;    // time lanes per conv block

template <typename T> __device__ __forceinline__ void store4(T* p, const f32x4& v);
template <> __device__ __forceinline__ void store4<float>(float* p, const f32x4& v) {
  *reinterpret_cast<f32x4*>(p) = v;
}
template <> __device__ __forceinline__ void store4<__bf16>(__bf16* p, const f32x4& v) {
  bf16x4 r = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
  *reinterpret_cast<bf16x4*>(p) = r;
}

// grid (ceil(C / 64) + 1, B), 256 threads. Blocks x < nsl: a slice of 64 conv channels of batch row b over all T
// tokens (thread = channel quad cq x time lane tl, tokens tl, tl + 16, ...), then the slice's conv state. Block
// x == nsl: the gate terms of row b. Each (b, channel) has a single owner block, so the state is read, and after a
// barrier rewritten, in place.
template <typename Tout>
__global__ __launch_bounds__(256) void gdn_conv_kernel(const float* __restrict__ y, int64_t ldy,
                                                       const float* __restrict__ cw, const float* __restrict__ cbias,
                                                       float* __restrict__ cstate, const float* __restrict__ A_log,
                                                       const float* __restrict__ dt_bias, int b_off, int a_off,
                                                       Tout* __restrict__ qo, Tout* __restrict__ ko,
                                                       Tout* __restrict__ vo, float* __restrict__ go,
                                                       float* __restrict__ betao, int T, int C, int Kd, int Vd,
                                                       int Hv, int K) {
  const int b = blockIdx.y, tid = threadIdx.x;
  const int nsl = (C + kConvCh - 1) / kConvCh;
  if ((int)blockIdx.x == nsl) {
    for (int i = tid; i < T * Hv; i += 256) {
      const int t = i / Hv, h = i - t * Hv;
      const float* row = y + ((int64_t)b * T + t) * ldy;
      const size_t oi = ((size_t)b * T + t) * Hv + h;
      betao[oi] = sigmoidf_(row[b_off + h]);
      go[oi] = -__expf(A_log[h]) * softplus_f(row[a_off + h] + dt_bias[h]);
    }
    return;
  }
  const int cq = tid & 15, tl = tid >> 4;
  const int c = kConvCh * blockIdx.x + 4 * cq;
  const bool cvalid = c < C;
  const int cc = cvalid ? c : C - 4;
  float w[4][kConvMaxK];
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int i = 0; i < kConvMaxK; ++i) w[e][i] = i < K ? cw[(size_t)(cc + e) * K + i] : 0.f;
  f32x4 bias = zero4();
  if (cbias) bias = *reinterpret_cast<const f32x4*>(cbias + cc);
  float* st = cstate + (size_t)b * (K - 1) * C;
  // output destination of this quad: q, k or v (a quad never straddles a boundary: Kd, Vd are multiples of 4)
  Tout* dst;
  int dstride, dcol;
  if (cc < Kd) { dst = qo; dstride = Kd; dcol = cc; }
  else if (cc < 2 * Kd) { dst = ko; dstride = Kd; dcol = cc - Kd; }
  else { dst = vo; dstride = Vd; dcol = cc - 2 * Kd; }
  for (int t = tl; t < T; t += kConvTl) {
    f32x4 acc = bias;
#pragma unroll
    for (int i = 0; i < kConvMaxK; ++i) {
      if (i >= K) break;
      const int ts = t - (K - 1) + i;  // input time of tap i
      const f32x4 x = ts >= 0 ? *reinterpret_cast<const f32x4*>(y + ((int64_t)b * T + ts) * ldy + cc)
                              : *reinterpret_cast<const f32x4*>(st + (size_t)(K - 1 + ts) * C + cc);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += w[e][i] * x[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = silu_f(acc[e]);
    if (cvalid) store4<Tout>(dst + ((size_t)b * T + t) * dstride + dcol, acc);
  }
  __syncthreads();
  // state <- the last K-1 entries of [old state | this call's inputs]; one thread per quad reads all its sources
  // before writing any slot
  if (tl == 0 && cvalid) {
    f32x4 nv[kConvMaxK - 1];
#pragma unroll
    for (int j = 0; j < kConvMaxK - 1; ++j) {
      if (j >= K - 1) break;
      const int src = T + j;  // index into [old (K-1) | inputs (T)]
      nv[j] = src >= K - 1 ? *reinterpret_cast<const f32x4*>(y + ((int64_t)b * T + src - (K - 1)) * ldy + c)
                           : *reinterpret_cast<const f32x4*>(st + (size_t)src * C + c);
    }
#pragma unroll
    for (int j = 0; j < kConvMaxK - 1; ++j) {
      if (j >= K - 1) break;
      *reinterpret_cast<f32x4*>(st + (size_t)j * C + c) = nv[j];
    }
  }
}

// T = 1 (the decode step): one thread per (row b, quad of 4 channels). Every load of the thread (taps, bias, the
// K-1 state rows, the input) is issued before any is used, and the thread owns its quad's state, so there is no
// barrier: one memory round trip. Block x == nb computes the gate terms of row b.
template <typename Tout>
__global__ __launch_bounds__(256) void gdn_conv1_kernel(const float* __restrict__ y, int64_t ldy,
                                                        const float* __restrict__ cw, const float* __restrict__ cbias,
                                                        float* __restrict__ cstate, const float* __restrict__ A_log,
                                                        const float* __restrict__ dt_bias, int b_off, int a_off,
                                                        Tout* __restrict__ qo, Tout* __restrict__ ko,
                                                        Tout* __restrict__ vo, float* __restrict__ go,
                                                        float* __restrict__ betao, int C, int Kd, int Vd, int Hv,
                                                        int K) {
  Q35_ARGS_UPFRONT(y, ldy, cw, cbias, cstate, A_log, dt_bias, b_off, a_off, qo, ko, vo, go, betao, C, Kd, Vd, Hv, K);
  const int b = blockIdx.y, tid = threadIdx.x;
  const int nb = (C / 4 + 255) / 256;
  const float* row = y + (int64_t)b * ldy;
  if ((int)blockIdx.x == nb) {
    for (int h = tid; h < Hv; h += 256) {
      betao[(size_t)b * Hv + h] = sigmoidf_(row[b_off + h]);
      go[(size_t)b * Hv + h] = -__expf(A_log[h]) * softplus_f(row[a_off + h] + dt_bias[h]);
    }
    return;
  }
  const int c = 4 * (blockIdx.x * 256 + tid);
  if (c >= C) return;
  float w[4][kConvMaxK];
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int i = 0; i < kConvMaxK; ++i) w[e][i] = i < K ? cw[(size_t)(c + e) * K + i] : 0.f;
  const f32x4 bias = cbias ? *reinterpret_cast<const f32x4*>(cbias + c) : zero4();
  float* st = cstate + (size_t)b * (K - 1) * C;
  f32x4 sx[kConvMaxK - 1];
#pragma unroll
  for (int j = 0; j < kConvMaxK - 1; ++j) sx[j] = j < K - 1 ? *reinterpret_cast<const f32x4*>(st + (size_t)j * C + c)
                                                           : zero4();
  const f32x4 xin = *reinterpret_cast<const f32x4*>(row + c);
  // tap i reads state row i for i < K - 1 and the input for i = K - 1
  f32x4 acc = bias;
#pragma unroll
  for (int i = 0; i < kConvMaxK; ++i) {
    if (i >= K) break;
    const f32x4 x = i < K - 1 ? sx[i] : xin;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += w[e][i] * x[e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = silu_f(acc[e]);
  Tout* dst;
  int dstride, dcol;
  if (c < Kd) { dst = qo; dstride = Kd; dcol = c; }
  else if (c < 2 * Kd) { dst = ko; dstride = Kd; dcol = c - Kd; }
  else { dst = vo; dstride = Vd; dcol = c - 2 * Kd; }
  store4<Tout>(dst + (size_t)b * dstride + dcol, acc);
  // state <- [old rows 1 .. K-2 | input]
#pragma unroll
  for (int j = 0; j < kConvMaxK - 1; ++j) {
    if (j >= K - 1) break;
    *reinterpret_cast<f32x4*>(st + (size_t)j * C + c) = j + 1 < K - 1 ? sx[j + 1] : xin;
  }
}

// One decode step (T = 1) of a Gated DeltaNet layer after its input projection, in one block of 1024 threads per
// (head h, row b), for Hk = Hv and dk = dv = 128: the q / k / v channels of head h through the causal conv + SiLU
// (their conv state advanced), beta and g, the recurrent update of the head's 128 x 128 fp32 state, and the gated
// RMSNorm of its output. The arithmetic and its reduction order are those of gdn_conv1_kernel, gdn_recurrent_kernel
// (T = 1) and gated_rmsnorm_kernel in fp32 (the results agree to rounding; a multiply-add may be contracted
// differently), and the conv state is advanced identically. The step saves two launches and the round trips of
// q, k, v, g, beta and o through memory.
// Threads 0..95 own one channel quad of the conv each (q, k, v: 32 quads each), thread 96 the gate terms. For the
// state, the block is four copies of gdn_recurrent_kernel's 256-thread layout, one per 32-column slice: thread t
// holds the float4 of columns 32 (t / 256) + 4 (t % 8) .. + 3 in rows (t % 256) / 8 + 32 i.
constexpr int kFD = 128;
__global__ __launch_bounds__(1024) void gdn_decode_fused_kernel(
    const float* __restrict__ y, int64_t ldy, const float* __restrict__ cw, const float* __restrict__ cbias,
    float* __restrict__ cstate, const float* __restrict__ A_log, const float* __restrict__ dt_bias, int b_off,
    int a_off, int z_off, float* __restrict__ S, const float* __restrict__ nw, const float* __restrict__ head_scale,
    float eps, float scale, float* __restrict__ out, int H, int C, int K) {
  Q35_ARGS_UPFRONT(y, ldy, cw, cbias, cstate, A_log, dt_bias, b_off, a_off, z_off, S, nw, head_scale, eps, scale, out,
                   H, C, K);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x, b = blockIdx.y;
  const float* row = y + (int64_t)b * ldy;
  __shared__ f32x4 vecs[3][kFD / 4];  // q, k, v of head h after the conv + SiLU
  __shared__ f32x4 red[16][8][2];     // [wave][column quad][S^T k | S^T q]
  __shared__ float ob[kFD];
  __shared__ float gates[2];          // beta, g

  // ---- 0. every load first: conv operands (threads 0..95), gate inputs (thread 96), the state slice, and the
  //         gated norm's z, w (wave 0)
  const bool conv_t = tid < 96;
  const int cr = tid >> 5, c4 = 4 * (tid & 31);
  const int ch = cr * H * kFD + h * kFD + c4;  // q: h D + c4, k: H D + h D + c4, v: 2 H D + h D + c4
  float w[4][kConvMaxK];
  f32x4 bias = zero4(), xin = zero4();
  f32x4 sx[kConvMaxK - 1];
  float* st = cstate + (size_t)b * (K - 1) * C;
  if (conv_t) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < kConvMaxK; ++i) w[e][i] = i < K ? cw[(size_t)(ch + e) * K + i] : 0.f;
    if (cbias) bias = *reinterpret_cast<const f32x4*>(cbias + ch);
#pragma unroll
    for (int j = 0; j < kConvMaxK - 1; ++j)
      sx[j] = j < K - 1 ? *reinterpret_cast<const f32x4*>(st + (size_t)j * C + ch) : zero4();
    xin = *reinterpret_cast<const f32x4*>(row + ch);
  }
  float gb = 0.f, ga = 0.f, gA = 0.f, gdt = 0.f;
  if (tid == 96) {
    gb = row[b_off + h];
    ga = row[a_off + h];
    gA = A_log[h];
    gdt = dt_bias[h];
  }
  const int sl = tid >> 8, tp = tid & 255, cq = tp & 7, rg = tp >> 3;
  const int j0 = 32 * sl + 4 * cq;
  float* sb = S + ((size_t)b * H + h) * kFD * kFD;
  f32x4 s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = *reinterpret_cast<const f32x4*>(sb + (size_t)(rg + 32 * i) * kFD + j0);
  float z0 = 0.f, z1 = 0.f, w0 = 0.f, w1 = 0.f, hs = 1.f;
  if (wave == 0) {
    z0 = row[z_off + h * kFD + 2 * lane];
    z1 = row[z_off + h * kFD + 2 * lane + 1];
    w0 = nw[2 * lane];
    w1 = nw[2 * lane + 1];
    if (head_scale) hs = head_scale[h];
  }

  // ---- 1. conv + SiLU (gdn_conv1_kernel's order), conv state <- [old rows 1 .. K-2 | input]; gate terms
  if (conv_t) {
    f32x4 acc = bias;
#pragma unroll
    for (int i = 0; i < kConvMaxK; ++i) {
      if (i >= K) break;
      const f32x4 x = i < K - 1 ? sx[i] : xin;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += w[e][i] * x[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = silu_f(acc[e]);
    vecs[cr][tid & 31] = acc;
#pragma unroll
    for (int j = 0; j < kConvMaxK - 1; ++j) {
      if (j >= K - 1) break;
      *reinterpret_cast<f32x4*>(st + (size_t)j * C + ch) = j + 1 < K - 1 ? sx[j + 1] : xin;
    }
  }
  if (tid == 96) {
    gates[0] = sigmoidf_(gb);
    gates[1] = -__expf(gA) * softplus_f(ga + gdt);
  }
  __syncthreads();

  // ---- 2. the recurrent step (gdn_recurrent_kernel's order): column sums of S k and S q over the slice's rows
  const float* qv = reinterpret_cast<const float*>(&vecs[0][0]);
  const float* kv = reinterpret_cast<const float*>(&vecs[1][0]);
  const float* vv = reinterpret_cast<const float*>(&vecs[2][0]);
  float kr[4], qr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kr[i] = kv[rg + 32 * i];
    qr[i] = qv[rg + 32 * i];
  }
  f32x4 a, c;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = s[0][e] * kr[0] + s[1][e] * kr[1] + s[2][e] * kr[2] + s[3][e] * kr[3];
    c[e] = s[0][e] * qr[0] + s[1][e] * qr[1] + s[2][e] * qr[2] + s[3][e] * qr[3];
  }
#pragma unroll
  for (int off = 8; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] += __shfl_xor(a[e], off, 64);
      c[e] += __shfl_xor(c[e], off, 64);
    }
  }
  if (lane < 8) {
    red[wave][lane][0] = a;
    red[wave][lane][1] = c;
  }
  const float q20 = qv[2 * lane], q21 = qv[2 * lane + 1], k20 = kv[2 * lane], k21 = kv[2 * lane + 1];
  float sq = q20 * q20 + q21 * q21;
  float sk = k20 * k20 + k21 * k21;
  float sqk = q20 * k20 + q21 * k21;
  sq = wave_sum(sq);
  sk = wave_sum(sk);
  sqk = wave_sum(sqk);
  __syncthreads();
  f32x4 A = red[4 * sl][cq][0], Cs = red[4 * sl][cq][1];
#pragma unroll
  for (int w2 = 1; w2 < 4; ++w2) {
    const f32x4 a2 = red[4 * sl + w2][cq][0], c2 = red[4 * sl + w2][cq][1];
#pragma unroll
    for (int e = 0; e < 4; ++e) { A[e] += a2[e]; Cs[e] += c2[e]; }
  }
  const float rk = rsqrtf(sk + 1e-6f);
  const float rqs = rsqrtf(sq + 1e-6f) * scale;
  const float qk = sqk * rqs * rk;
  const float beta = gates[0], alpha = expf(gates[1]);
  float kk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) kk[i] = kr[i] * rk;
  f32x4 o4;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float d = beta * (vv[j0 + e] - alpha * rk * A[e]);
    o4[e] = alpha * rqs * Cs[e] + qk * d;
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i][e] = alpha * s[i][e] + kk[i] * d;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<f32x4*>(sb + (size_t)(rg + 32 * i) * kFD + j0) = s[i];
  if (rg == 0) *reinterpret_cast<f32x4*>(&ob[j0]) = o4;
  __syncthreads();

  // ---- 3. gated RMSNorm of the head's output (gated_rmsnorm_kernel's order)
  if (wave == 0) {
    const float x0 = ob[2 * lane], x1 = ob[2 * lane + 1];
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float r = rsqrtf(ss * (1.f / 128.f) + eps);
    const float n0 = x0 * r, n1 = x1 * r;
    float* orw = out + ((size_t)b * H + h) * kFD;
    orw[2 * lane] = w0 * n0 * silu_f(z0) * hs;
    orw[2 * lane + 1] = w1 * n1 * silu_f(z1) * hs;
  }
}

// The recurrent part of a GDN decode step (T = 1), split over four blocks of 256 threads per (head h, row b), for
// Hk = Hv and dk = dv = 128, after an input projection whose epilogue already ran the causal conv + SiLU
// (q35_gemv_norm_conv): q, k, v of head h are read straight from the projection row y. Block (j, h, b) updates
// state columns 32 j .. 32 j + 31 with gdn_recurrent_kernel's thread layout (slice j of the fused kernel, so the
// column sums are formed in the same order), computes beta and g from the row's b and a columns, and writes those
// 32 columns of the head's raw output o; the gated RMSNorm is left to the output projection (q35_gemv_gated_norm).
// 192 blocks at B 3, H 16 against the fused kernel's 48: a quarter of the state bytes per CU.
__global__ __launch_bounds__(256) void gdn_decode_sliced_kernel(
    const float* __restrict__ y, int64_t ldy, const float* __restrict__ A_log, const float* __restrict__ dt_bias,
    int b_off, int a_off, float* __restrict__ S, float scale, float* __restrict__ out, int H) {
  Q35_ARGS_UPFRONT(y, ldy, A_log, dt_bias, b_off, a_off, S, scale, out, H);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sj = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const float* row = y + (int64_t)b * ldy;
  __shared__ f32x4 red[4][8][2];  // [wave][column quad][S^T k | S^T q]
  __shared__ float gates[2];      // beta, g

  // ---- 0. every load first: the state slice, this thread's q and k rows, the lane pairs of q and k for the norms,
  //         the column quad of v, the gate inputs (thread 0)
  const int cq = tid & 7, rg = tid >> 3;
  const int j0 = 32 * sj + 4 * cq;
  float* sb = S + ((size_t)b * H + h) * kFD * kFD;
  f32x4 s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = *reinterpret_cast<const f32x4*>(sb + (size_t)(rg + 32 * i) * kFD + j0);
  const float* qv = row + (size_t)h * kFD;
  const float* kv = row + (size_t)(H + h) * kFD;
  const float* vv = row + (size_t)(2 * H + h) * kFD;
  float kr[4], qr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kr[i] = kv[rg + 32 * i];
    qr[i] = qv[rg + 32 * i];
  }
  const float q20 = qv[2 * lane], q21 = qv[2 * lane + 1], k20 = kv[2 * lane], k21 = kv[2 * lane + 1];
  const f32x4 v4 = *reinterpret_cast<const f32x4*>(vv + j0);
  float gb = 0.f, ga = 0.f, gA = 0.f, gdt = 0.f;
  if (tid == 0) {
    gb = row[b_off + h];
    ga = row[a_off + h];
    gA = A_log[h];
    gdt = dt_bias[h];
  }

  // ---- 1. column sums of S k and S q over the slice's rows (the fused kernel's order), the norms, the gates
  f32x4 a, c;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = s[0][e] * kr[0] + s[1][e] * kr[1] + s[2][e] * kr[2] + s[3][e] * kr[3];
    c[e] = s[0][e] * qr[0] + s[1][e] * qr[1] + s[2][e] * qr[2] + s[3][e] * qr[3];
  }
#pragma unroll
  for (int off = 8; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] += __shfl_xor(a[e], off, 64);
      c[e] += __shfl_xor(c[e], off, 64);
    }
  }
  if (lane < 8) {
    red[wave][lane][0] = a;
    red[wave][lane][1] = c;
  }
  if (tid == 0) {
    gates[0] = sigmoidf_(gb);
    gates[1] = -__expf(gA) * softplus_f(ga + gdt);
  }
  float sq = q20 * q20 + q21 * q21;
  float sk = k20 * k20 + k21 * k21;
  float sqk = q20 * k20 + q21 * k21;
  sq = wave_sum(sq);
  sk = wave_sum(sk);
  sqk = wave_sum(sqk);
  __syncthreads();

  // ---- 2. the update of the slice and its 32 output columns
  f32x4 A = red[0][cq][0], Cs = red[0][cq][1];
#pragma unroll
  for (int w2 = 1; w2 < 4; ++w2) {
    const f32x4 a2 = red[w2][cq][0], c2 = red[w2][cq][1];
#pragma unroll
    for (int e = 0; e < 4; ++e) { A[e] += a2[e]; Cs[e] += c2[e]; }
  }
  const float rk = rsqrtf(sk + 1e-6f);
  const float rqs = rsqrtf(sq + 1e-6f) * scale;
  const float qk = sqk * rqs * rk;
  const float beta = gates[0], alpha = expf(gates[1]);
  float kk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) kk[i] = kr[i] * rk;
  f32x4 o4;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float d = beta * (v4[e] - alpha * rk * A[e]);
    o4[e] = alpha * rqs * Cs[e] + qk * d;
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i][e] = alpha * s[i][e] + kk[i] * d;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<f32x4*>(sb + (size_t)(rg + 32 * i) * kFD + j0) = s[i];
  if (rg == 0) *reinterpret_cast<f32x4*>(out + ((size_t)b * H + h) * kFD + j0) = o4;
}

// One wave per (token m, head h) of o [M, Hv, dv]; dv = 128 (two values per lane). Four waves per block.
// XS (fp32 o): out in the int8 GEMM's split layout (each group of 8 values as 8 bf16 hi parts, then 8 bf16 lo parts),
// the output projection's input read without splitting.
template <typename T, bool XS>
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const T* __restrict__ o, const float* __restrict__ z,
                                                            int64_t ldz, const float* __restrict__ w,
                                                            const float* __restrict__ head_scale, T* __restrict__ out,
                                                            int64_t M, int Hv, float eps) {
  Q35_ARGS_UPFRONT(o, z, ldz, w, head_scale, out, M, Hv, eps);
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (job >= M * Hv) return;
  const int64_t m = job / Hv;
  const int h = (int)(job - m * Hv);
  const T* orow = o + job * 128;
  const float x0 = to_f32(orow[2 * lane]), x1 = to_f32(orow[2 * lane + 1]);
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float r = rsqrtf(ss * (1.f / 128.f) + eps);
  const float* zr = z + m * ldz + h * 128;
  const float hs = head_scale ? head_scale[h] : 1.f;
  // HF rounds the normalised value to the input dtype before the weight multiply
  const float n0 = to_f32(from_f32<T>(x0 * r)), n1 = to_f32(from_f32<T>(x1 * r));
  T* orw = out + job * 128;
  const float y0 = w[2 * lane] * n0 * silu_f(zr[2 * lane]) * hs;
  const float y1 = w[2 * lane + 1] * n1 * silu_f(zr[2 * lane + 1]) * hs;
  if constexpr (XS) {  // values 2 l, 2 l + 1: positions 2 (l % 4) .. + 1 of group l / 4
    __bf16* g = reinterpret_cast<__bf16*>(orw + 8 * (lane >> 2));
    const bf16_hl a = bf16_split(y0), c = bf16_split(y1);
    const int e = 2 * (lane & 3);
    g[e] = a.hi;
    g[e + 1] = c.hi;
    g[8 + e] = a.lo;
    g[9 + e] = c.lo;
  } else {
    orw[2 * lane] = from_f32<T>(y0);
    orw[2 * lane + 1] = from_f32<T>(y1);
  }
}

// The same norm with 16-byte accesses (o, z, w, out 16-byte aligned, ldz a multiple of 4): two (token, head) jobs per
// wave, 32 lanes per job, four values per lane; the squares are summed over the 32 lanes with xor shuffles. The
// arithmetic per value is gated_rmsnorm_kernel's (only the summation order of the squares differs).
template <typename T, bool XS>
__global__ __launch_bounds__(256) void gated_rmsnorm4_kernel(const T* __restrict__ o, const float* __restrict__ z,
                                                             int64_t ldz, const float* __restrict__ w,
                                                             const float* __restrict__ head_scale,
                                                             T* __restrict__ out, int64_t M, int Hv, float eps) {
  Q35_ARGS_UPFRONT(o, z, ldz, w, head_scale, out, M, Hv, eps);
  const int lane = threadIdx.x & 63, hl = lane & 31;
  const int64_t job = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 2 + (lane >> 5);
  if (job >= M * Hv) return;  // whole halves only: the shuffles below stay inside a half
  const int64_t m = job / Hv;
  const int h = (int)(job - m * Hv);
  float x[4];
  if constexpr (std::is_same<T, float>::value) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(o + job * 128 + 4 * hl);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = t[e];
  } else {
    const bf16x4 t = *reinterpret_cast<const bf16x4*>(o + job * 128 + 4 * hl);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = (float)t[e];
  }
  float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) ss += __shfl_xor(ss, off, 64);
  const float r = rsqrtf(ss * (1.f / 128.f) + eps);
  const f32x4 zz = *reinterpret_cast<const f32x4*>(z + m * ldz + h * 128 + 4 * hl);
  const f32x4 ww = *reinterpret_cast<const f32x4*>(w + 4 * hl);
  const float hs = head_scale ? head_scale[h] : 1.f;
  float y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float n = to_f32(from_f32<T>(x[e] * r));  // HF rounds the normalised value to the input dtype
    y[e] = ww[e] * n * silu_f(zz[e]) * hs;
  }
  T* orw = out + job * 128;
  if constexpr (XS) {  // values 4 l .. 4 l + 3: half l % 2 of group l / 2 (8 bytes of its hi and of its lo part)
    bf16x4 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bf16_hl t = bf16_split(y[e]);
      hi[e] = t.hi;
      lo[e] = t.lo;
    }
    float* gp = reinterpret_cast<float*>(orw) + 8 * (hl >> 1) + 2 * (hl & 1);
    *reinterpret_cast<bf16x4*>(gp) = hi;
    *reinterpret_cast<bf16x4*>(gp + 4) = lo;
  } else if constexpr (std::is_same<T, float>::value) {
    *reinterpret_cast<f32x4*>(orw + 4 * hl) = f32x4{y[0], y[1], y[2], y[3]};
  } else {
    bf16x4 t;
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = (__bf16)y[e];
    *reinterpret_cast<bf16x4*>(orw + 4 * hl) = t;
  }
}

// One wave per (token m, job j) with j < Hq: query head j; Hq <= j < Hq + Hkv: key head; then value heads.
// D = 256: four values per lane (dims 4 l .. 4 l + 3). Four waves per block.
__global__ __launch_bounds__(256) void attn_prep_kernel(const float* __restrict__ y, int64_t ldy,
                                                        const float* __restrict__ qw, const float* __restrict__ kw,
                                                        float eps, const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, int rot,
                                                        const int32_t* __restrict__ pos, __bf16* __restrict__ q_out,
                                                        __bf16* __restrict__ gate_out, __bf16* __restrict__ k_out,
                                                        __bf16* __restrict__ v_out, __bf16* __restrict__ k_cache,
                                                        __bf16* __restrict__ v_cache, int max_len, int T, int Hq,
                                                        int Hkv, int64_t M) {
  Q35_ARGS_UPFRONT(y, ldy, qw, kw, eps, cos_t, sin_t, rot, pos, q_out, gate_out, k_out, v_out, k_cache, v_cache,
                   max_len, T, Hq, Hkv, M);
  constexpr int D = 256;
  const int lane = threadIdx.x & 63;
  const int jobs = Hq + 2 * Hkv;
  const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= M * jobs) return;
  const int64_t m = g / jobs;
  const int j = (int)(g - m * jobs);
  const int b = (int)(m / T), t = (int)(m - (int64_t)b * T);
  const float* row = y + m * ldy;
  const int d0 = 4 * lane;
  if (j < Hq) {  // query head j: normalise q, copy the gate half
    const f32x4 x = *reinterpret_cast<const f32x4*>(row + (size_t)j * 2 * D + d0);
    const f32x4 gt = *reinterpret_cast<const f32x4*>(row + (size_t)j * 2 * D + D + d0);
    const float ss = wave_sum(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
    const float r = rsqrtf(ss * (1.f / D) + eps);
    const f32x4 wv = *reinterpret_cast<const f32x4*>(qw + d0);
    f32x4 qn;
#pragma unroll
    for (int e = 0; e < 4; ++e) qn[e] = x[e] * r * (1.f + wv[e]);
    store4<__bf16>(q_out + (m * Hq + j) * D + d0, qn);
    store4<__bf16>(gate_out + (m * Hq + j) * D + d0, gt);
    return;
  }
  const int p = min(max(pos[b], 0), max_len) + t;  // absolute position of this token
  if (j < Hq + Hkv) {  // key head
    const int kh = j - Hq;
    const f32x4 x = *reinterpret_cast<const f32x4*>(row + (size_t)Hq * 2 * D + (size_t)kh * D + d0);
    const float ss = wave_sum(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
    const float r = rsqrtf(ss * (1.f / D) + eps);
    const f32x4 wv = *reinterpret_cast<const f32x4*>(kw + d0);
    f32x4 kn;
#pragma unroll
    for (int e = 0; e < 4; ++e) kn[e] = x[e] * r * (1.f + wv[e]);
    if (k_out) store4<__bf16>(k_out + (m * Hkv + kh) * D + d0, kn);
    // rotate-half partner of dims d0..d0+3 (d < rot): d +- rot/2, held by lane l +- rot/8
    const int half = rot >> 1;
    const int pl = d0 < half ? lane + half / 4 : lane - half / 4;
    f32x4 pn;
#pragma unroll
    for (int e = 0; e < 4; ++e) pn[e] = __shfl(kn[e], d0 < rot ? pl : lane, 64);
    if (p < max_len) {
      f32x4 kr = kn;
      if (d0 < rot) {
        const int j0 = d0 < half ? d0 : d0 - half;
        const f32x4 cv = *reinterpret_cast<const f32x4*>(cos_t + (size_t)p * half + j0);
        const f32x4 sv = *reinterpret_cast<const f32x4*>(sin_t + (size_t)p * half + j0);
        const float sg = d0 < half ? -1.f : 1.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) kr[e] = kn[e] * cv[e] + sg * pn[e] * sv[e];
      }
      store4<__bf16>(k_cache + (((size_t)b * Hkv + kh) * max_len + p) * D + d0, kr);
    }
    return;
  }
  const int vh = j - Hq - Hkv;  // value head
  const f32x4 x = *reinterpret_cast<const f32x4*>(row + (size_t)Hq * 2 * D + (size_t)(Hkv + vh) * D + d0);
  if (v_out) store4<__bf16>(v_out + (m * Hkv + vh) * D + d0, x);
  if (p < max_len) store4<__bf16>(v_cache + (((size_t)b * Hkv + vh) * max_len + p) * D + d0, x);
}

// Residual add + RMSNorm with (1 + w) (HF:720-734 Qwen3_5RMSNorm, applied around every mixer and MLP at HF:753-793;
// engine/kernels.js:226-246 `rmsnorm` with OFFSET and `addInto`): x[m] += y[m] (when y is given) in place, then
// h[m] = x[m] * rsqrt(mean(x[m]^2) + eps) * (1 + w), all fp32. One block of 256 threads per row; H a multiple of 4.
// XS: h in the int8 GEMM's split layout instead (each group of 8 inputs as 8 bf16 hi parts, then 8 bf16 lo parts,
// hi = bf16(h), lo = bf16(h - hi); H a multiple of 8), the form q35_gemm_q8_split reads without splitting.
template <bool XS>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(float* __restrict__ x, int64_t ldx,
                                                          const float* __restrict__ y, int64_t ldy,
                                                          const float* __restrict__ w, float* __restrict__ h,
                                                          int64_t ldh, int H, float eps) {
  Q35_ARGS_UPFRONT(x, ldx, y, ldy, w, h, ldh, H, eps);
  const int64_t m = blockIdx.x;
  const int tid = threadIdx.x;
  float* xr = x + m * ldx;
  const float* yr = y ? y + m * ldy : nullptr;
  constexpr int kMaxPer = 8;  // float4s per thread held in registers (H <= 8192)
  f32x4 v[kMaxPer];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int c = 4 * (tid + 256 * i);
    if (c < H) {
      v[i] = *reinterpret_cast<const f32x4*>(xr + c);
      if (yr) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(yr + c);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i][e] += a[e];
        *reinterpret_cast<f32x4*>(xr + c) = v[i];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) ss += v[i][e] * v[i][e];
    }
  }
  __shared__ float red[4];
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float r = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + eps);
  float* hr = h + m * ldh;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int c = 4 * (tid + 256 * i);
    if (c < H) {
      const f32x4 wv = *reinterpret_cast<const f32x4*>(w + c);
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = v[i][e] * r * (1.f + wv[e]);
      if constexpr (XS) {  // inputs c .. c + 3: half (c / 4) % 2 of group c / 8 (8 bytes of its hi and of its lo part)
        bf16x4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bf16_hl t = bf16_split(o[e]);
          hi[e] = t.hi;
          lo[e] = t.lo;
        }
        float* gp = hr + 8 * (c >> 3) + 2 * ((c >> 2) & 1);
        *reinterpret_cast<bf16x4*>(gp) = hi;
        *reinterpret_cast<bf16x4*>(gp + 4) = lo;
      } else {
        *reinterpret_cast<f32x4*>(hr + c) = o;
      }
    }
  }
}

}  // namespace q35

namespace q35 {

template <bool XS>
static int add_rmsnorm_run(float* x, int64_t ldx, const float* y, int64_t ldy, const float* w, float* h, int64_t ldh,
                           int64_t M, int64_t H, float eps, q35_stream_t stream) {
  if (!x || !w || !h || M <= 0 || H <= 0 || ldx < H || ldh < H || (y && ldy < H)) return Q35_EINVAL;
  if ((H & 3) || H > 8192 || (ldx & 3) || (ldh & 3) || (y && (ldy & 3)) || M > 0x7fffffff) return Q35_EUNSUPPORTED;
  if (XS && (H & 7)) return Q35_EUNSUPPORTED;
  if (((uintptr_t)x & 15) || ((uintptr_t)h & 15) || ((uintptr_t)w & 15) || (y && ((uintptr_t)y & 15)))
    return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(add_rmsnorm_kernel<XS>, dim3((unsigned)M), dim3(256), 0, st, x, ldx, y, ldy, w, h, ldh, (int)H,
                     eps);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

}  // namespace q35

extern "C" int q35_add_rmsnorm(float* x, int64_t ldx, const float* y, int64_t ldy, const float* w, float* h,
                               int64_t ldh, int64_t M, int64_t H, float eps, q35_stream_t stream) {
  return q35::add_rmsnorm_run<false>(x, ldx, y, ldy, w, h, ldh, M, H, eps, stream);
}

extern "C" int q35_add_rmsnorm_split(float* x, int64_t ldx, const float* y, int64_t ldy, const float* w, void* hs,
                                     int64_t ldh, int64_t M, int64_t H, float eps, q35_stream_t stream) {
  return q35::add_rmsnorm_run<true>(x, ldx, y, ldy, w, static_cast<float*>(hs), ldh, M, H, eps, stream);
}

extern "C" int q35_gdn_decode_fused(const float* y, int64_t ldy, const float* conv_w, const float* conv_bias,
                                    float* conv_state, const float* A_log, const float* dt_bias, int64_t b_off,
                                    int64_t a_off, int64_t z_off, float* state, const float* norm_w,
                                    const float* head_scale, float eps, float scale, float* out, int64_t B, int64_t H,
                                    int64_t d, int64_t K, q35_stream_t stream) {
  using namespace q35;
  if (!y || !conv_w || !conv_state || !A_log || !dt_bias || !state || !norm_w || !out) return Q35_EINVAL;
  if (B <= 0 || H <= 0 || d <= 0 || K < 2) return Q35_EINVAL;
  const int64_t C = 3 * H * d, Vd = H * d;
  if (ldy < C || b_off < 0 || a_off < 0 || z_off < 0 || b_off + H > ldy || a_off + H > ldy || z_off + Vd > ldy)
    return Q35_EINVAL;
  if (d != kFD || K > kConvMaxK || (ldy & 3) || ((uintptr_t)y & 15) || ((uintptr_t)conv_state & 15) ||
      ((uintptr_t)state & 15))
    return Q35_EUNSUPPORTED;
  if (conv_bias && ((uintptr_t)conv_bias & 15)) return Q35_EUNSUPPORTED;
  if (B > 65535 || H > 65535 || B * ldy > ((int64_t)1 << 40) || C > 0x7fffffff) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gdn_decode_fused_kernel, dim3((unsigned)H, (unsigned)B), dim3(1024), 0, st, y, ldy, conv_w,
                     conv_bias, conv_state, A_log, dt_bias, (int)b_off, (int)a_off, (int)z_off, state, norm_w,
                     head_scale, eps, scale, out, (int)H, (int)C, (int)K);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

extern "C" int q35_gdn_decode_sliced(const float* y, int64_t ldy, const float* A_log, const float* dt_bias,
                                     int64_t b_off, int64_t a_off, float* state, float scale, float* out, int64_t B,
                                     int64_t H, int64_t d, q35_stream_t stream) {
  using namespace q35;
  if (!y || !A_log || !dt_bias || !state || !out) return Q35_EINVAL;
  if (B <= 0 || H <= 0 || d <= 0) return Q35_EINVAL;
  const int64_t C = 3 * H * d;
  if (ldy < C || b_off < 0 || a_off < 0 || b_off + H > ldy || a_off + H > ldy) return Q35_EINVAL;
  if (d != kFD || (ldy & 3) || ((uintptr_t)y & 15) || ((uintptr_t)state & 15) || ((uintptr_t)out & 15))
    return Q35_EUNSUPPORTED;
  if (B > 65535 || H > 65535 || B * ldy > ((int64_t)1 << 40)) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gdn_decode_sliced_kernel, dim3(4, (unsigned)H, (unsigned)B), dim3(256), 0, st, y, ldy, A_log,
                     dt_bias, (int)b_off, (int)a_off, state, scale, out, (int)H);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

extern "C" int q35_gdn_conv(const float* y, int64_t ldy, const float* conv_w, const float* conv_bias,
                            float* conv_state, const float* A_log, const float* dt_bias, int64_t b_off, int64_t a_off,
                            void* q, void* k, void* v, float* g, float* beta, int64_t B, int64_t T, int64_t Hk,
                            int64_t dk, int64_t Hv, int64_t dv, int64_t K, int dtype, q35_stream_t stream) {
  using namespace q35;
  if (!y || !conv_w || !conv_state || !A_log || !dt_bias || !q || !k || !v || !g || !beta) return Q35_EINVAL;
  if (B <= 0 || T <= 0 || Hk <= 0 || dk <= 0 || Hv <= 0 || dv <= 0 || K < 2) return Q35_EINVAL;
  const int64_t Kd = Hk * dk, Vd = Hv * dv, C = 2 * Kd + Vd;
  if (ldy < C || b_off < 0 || a_off < 0 || b_off + Hv > ldy || a_off + Hv > ldy) return Q35_EINVAL;
  if (K > kConvMaxK || (Kd & 3) || (Vd & 3) || (ldy & 3) || ((uintptr_t)y & 15) || ((uintptr_t)conv_state & 15))
    return Q35_EUNSUPPORTED;
  if (conv_bias && ((uintptr_t)conv_bias & 15)) return Q35_EUNSUPPORTED;
  if (B > 65535 || B * T * ldy > ((int64_t)1 << 40) || T * Hv > 0x7fffffff || C > 0x7fffffff)
    return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (T == 1) {  // decode: one thread per channel quad
    const dim3 g1((unsigned)((C / 4 + 255) / 256 + 1), (unsigned)B);
    if (dtype == Q35_F32)
      hipLaunchKernelGGL(gdn_conv1_kernel<float>, g1, dim3(256), 0, st, y, ldy, conv_w, conv_bias, conv_state, A_log,
                         dt_bias, (int)b_off, (int)a_off, (float*)q, (float*)k, (float*)v, g, beta, (int)C, (int)Kd,
                         (int)Vd, (int)Hv, (int)K);
    else if (dtype == Q35_BF16)
      hipLaunchKernelGGL(gdn_conv1_kernel<__bf16>, g1, dim3(256), 0, st, y, ldy, conv_w, conv_bias, conv_state,
                         A_log, dt_bias, (int)b_off, (int)a_off, (__bf16*)q, (__bf16*)k, (__bf16*)v, g, beta, (int)C,
                         (int)Kd, (int)Vd, (int)Hv, (int)K);
    else
      return Q35_EUNSUPPORTED;
    return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
  }
  const dim3 grid((unsigned)((C + kConvCh - 1) / kConvCh + 1), (unsigned)B);
  if (dtype == Q35_F32)
    hipLaunchKernelGGL(gdn_conv_kernel<float>, grid, dim3(256), 0, st, y, ldy, conv_w, conv_bias, conv_state, A_log,
                       dt_bias, (int)b_off, (int)a_off, (float*)q, (float*)k, (float*)v, g, beta, (int)T, (int)C,
                       (int)Kd, (int)Vd, (int)Hv, (int)K);
  else if (dtype == Q35_BF16)
    hipLaunchKernelGGL(gdn_conv_kernel<__bf16>, grid, dim3(256), 0, st, y, ldy, conv_w, conv_bias, conv_state,
                       A_log, dt_bias, (int)b_off, (int)a_off, (__bf16*)q, (__bf16*)k, (__bf16*)v, g, beta, (int)T,
                       (int)C, (int)Kd, (int)Vd, (int)Hv, (int)K);
  else
    return Q35_EUNSUPPORTED;
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

extern "C" int q35_gated_rmsnorm(const void* o, const float* z, int64_t ldz, const float* w, const float* head_scale,
                                 void* out, int64_t M, int64_t Hv, int64_t dv, float eps, int dtype,
                                 q35_stream_t stream) {
  using namespace q35;
  if (!o || !z || !w || !out || M <= 0 || Hv <= 0 || dv <= 0 || ldz < Hv * dv) return Q35_EINVAL;
  if (dv != 128) return Q35_EUNSUPPORTED;
  const int64_t blocks = (M * Hv + 3) / 4;
  if (blocks > 0x7fffffff) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool v4 = !(((uintptr_t)o | (uintptr_t)z | (uintptr_t)w | (uintptr_t)out) & 15) && ldz % 4 == 0;
  const unsigned blocks4 = (unsigned)((M * Hv + 7) / 8);
  if (v4 && dtype == Q35_F32)
    hipLaunchKernelGGL((gated_rmsnorm4_kernel<float, false>), dim3(blocks4), dim3(256), 0, st, (const float*)o, z, ldz,
                       w, head_scale, (float*)out, M, (int)Hv, eps);
  else if (v4 && dtype == Q35_BF16)
    hipLaunchKernelGGL((gated_rmsnorm4_kernel<__bf16, false>), dim3(blocks4), dim3(256), 0, st, (const __bf16*)o, z,
                       ldz, w, head_scale, (__bf16*)out, M, (int)Hv, eps);
  else if (dtype == Q35_F32)
    hipLaunchKernelGGL((gated_rmsnorm_kernel<float, false>), dim3((unsigned)blocks), dim3(256), 0, st, (const float*)o, z,
                       ldz, w, head_scale, (float*)out, M, (int)Hv, eps);
  else if (dtype == Q35_BF16)
    hipLaunchKernelGGL((gated_rmsnorm_kernel<__bf16, false>), dim3((unsigned)blocks), dim3(256), 0, st, (const __bf16*)o, z,
                       ldz, w, head_scale, (__bf16*)out, M, (int)Hv, eps);
  else
    return Q35_EUNSUPPORTED;
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

extern "C" int q35_gated_rmsnorm_split(const float* o, const float* z, int64_t ldz, const float* w,
                                       const float* head_scale, void* out, int64_t M, int64_t Hv, int64_t dv, float eps,
                                       q35_stream_t stream) {
  using namespace q35;
  if (!o || !z || !w || !out || M <= 0 || Hv <= 0 || dv <= 0 || ldz < Hv * dv) return Q35_EINVAL;
  if (dv != 128 || ((uintptr_t)out & 15)) return Q35_EUNSUPPORTED;
  const int64_t blocks = (M * Hv + 3) / 4;
  if (blocks > 0x7fffffff) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!(((uintptr_t)o | (uintptr_t)z | (uintptr_t)w) & 15) && ldz % 4 == 0)
    hipLaunchKernelGGL((gated_rmsnorm4_kernel<float, true>), dim3((unsigned)((M * Hv + 7) / 8)), dim3(256), 0, st, o, z,
                       ldz, w, head_scale, static_cast<float*>(out), M, (int)Hv, eps);
  else
    hipLaunchKernelGGL((gated_rmsnorm_kernel<float, true>), dim3((unsigned)blocks), dim3(256), 0, st, o, z, ldz, w,
                       head_scale, static_cast<float*>(out), M, (int)Hv, eps);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

extern "C" int q35_attn_prep(const float* y, int64_t ldy, const float* q_norm_w, const float* k_norm_w, float eps,
                             const float* cos, const float* sin, int64_t rot, const int32_t* pos, void* q_out,
                             void* gate_out, void* k_out, void* v_out, void* k_cache, void* v_cache, int64_t max_len,
                             int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, q35_stream_t stream) {
  using namespace q35;
  if (!y || !q_norm_w || !k_norm_w || !pos || !q_out || !gate_out || !k_cache || !v_cache) return Q35_EINVAL;
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_len <= 0 || rot < 0 || rot > D) return Q35_EINVAL;
  if (ldy < 2 * Hq * D + 2 * Hkv * D) return Q35_EINVAL;
  if (rot > 0 && (!cos || !sin)) return Q35_EINVAL;
  if (D != 256 || (rot % 8) != 0 || (ldy & 3) || ((uintptr_t)y & 15)) return Q35_EUNSUPPORTED;
  const int64_t M = B * T;
  const int64_t blocks = (M * (Hq + 2 * Hkv) + 3) / 4;
  if (blocks > 0x7fffffff || max_len > 0x7fffffff || T > 0x7fffffff) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)blocks), dim3(256), 0, st, y, ldy, q_norm_w, k_norm_w, eps, cos,
                     sin, (int)rot, pos, (__bf16*)q_out, (__bf16*)gate_out, (__bf16*)k_out, (__bf16*)v_out,
                     (__bf16*)k_cache, (__bf16*)v_cache, (int)max_len, (int)T, (int)Hq, (int)Hkv, M);
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
