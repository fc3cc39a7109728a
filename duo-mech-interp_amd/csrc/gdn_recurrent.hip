// Gated DeltaNet, token-serial form: the decode step (and any T, with the state kept in registers across tokens).
//
// Per (batch b, value head h) and token t, with the state S[Dk][Dv] in fp32 (HF:331-380; WGSL engine/kernels_qwen35.js
// :209-236):
//   q, k  <- optional l2norm (x * rsqrt(sum x^2 + 1e-6), HF:242-245), q *= scale
//   S     <- exp(g_t) * S
//   u_j    = sum_i S[i][j] k_i                  (kv_mem, HF:370)
//   d_j    = beta_t (v_j - u_j)
//   S     <- S + k d^T
//   o_j    = sum_i S[i][j] q_i
// The kernel reads S once and writes it once per launch: with a = S^T k and c = S^T q taken on the undecayed S,
//   u = alpha a,  o = alpha c + (q . k) d,  S' = alpha S + k d^T,
// which is the same arithmetic regrouped (both dot products come from one pass over the state tile). The norms are
// folded in as scalars: a and c are taken with the raw k and q and scaled by rsqrt(|k|^2 + eps) and
// rsqrt(|q|^2 + eps) * scale afterwards.
//
// Decomposition: value columns are independent given k and q, so one block of 256 threads takes a slice of 32 value
// columns (128 bytes of every state row, one full cache line) of one (head, row): grid (Dv / 32, H, B). Thread t
// owns the float4 of columns 4 (t % 8) .. + 3 in the four rows t / 8 + 32 i, so one wave load covers eight whole
// 128-byte lines. Column sums run as three xor-shuffles over the lanes of a wave with equal t % 8, then across the
// four waves through LDS (double-buffered by token parity: one barrier per token). Every wave forms |q|^2, |k|^2
// and q . k itself from two elements per lane, and the next token's inputs are loaded while the current token is
// reduced, so a token costs one barrier and no exposed global-load latency after the first.
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kGdnD = 128;   // Dk = Dv
constexpr int kGdnJS = 32;   // value columns per block

// Per-token inputs of one thread (loaded one token ahead).
struct RecIn {
  float kr[4], qr[4];  // k and q at this thread's four state rows
  float k2[2], q2[2];  // two elements per lane for the norms
  float vv[4];         // v at this thread's four value columns
  float g, beta;
};

template <typename Tin>
__device__ __forceinline__ void rec_load(RecIn& in, const Tin* __restrict__ q, const Tin* __restrict__ k,
                                         const Tin* __restrict__ v, const float* __restrict__ g,
                                         const float* __restrict__ beta, size_t tok, int Hk, int kh, int H, int h,
                                         int rg, int j0, int lane) {
  const Tin* qrow = q + (tok * Hk + kh) * kGdnD;
  const Tin* krow = k + (tok * Hk + kh) * kGdnD;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    in.kr[i] = to_f32(krow[rg + 32 * i]);
    in.qr[i] = to_f32(qrow[rg + 32 * i]);
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    in.k2[e] = to_f32(krow[2 * lane + e]);
    in.q2[e] = to_f32(qrow[2 * lane + e]);
  }
  const Tin* vrow = v + (tok * H + h) * kGdnD + j0;
#pragma unroll
  for (int e = 0; e < 4; ++e) in.vv[e] = to_f32(vrow[e]);
  in.g = g[tok * H + h];
  in.beta = beta[tok * H + h];
}

template <typename Tin>
__global__ __launch_bounds__(256) void gdn_recurrent_kernel(const Tin* __restrict__ q, const Tin* __restrict__ k,
                                                            const Tin* __restrict__ v, const float* __restrict__ g,
                                                            const float* __restrict__ beta, const float* s_in,
                                                            float* s_out, Tin* __restrict__ o, int T, int Hk, int H,
                                                            float scale, int l2norm) {
  Q35_ARGS_UPFRONT(q, k, v, g, beta, s_in, s_out, o, T, Hk, H, scale, l2norm);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int cq = tid & 7;   // column quad of this thread
  const int rg = tid >> 3;  // rows rg + 32 i
  const int j0 = blockIdx.x * kGdnJS + cq * 4;
  const int h = blockIdx.y, b = blockIdx.z;
  const int kh = h / (H / Hk);

  __shared__ f32x4 red[2][4][8][2];  // [token parity][wave][column quad][S^T k | S^T q]

  // The first token's inputs are loaded before the state: issued after it, they would queue behind every block's
  // state reads at the memory controllers, and nothing can be computed without them.
  RecIn cur, nxt;
  rec_load(cur, q, k, v, g, beta, (size_t)b * T, Hk, kh, H, h, rg, j0, lane);
  asm volatile("" ::: "memory");
  const size_t sbase = ((size_t)b * H + h) * kGdnD * kGdnD;
  f32x4 s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    s[i] = s_in ? *reinterpret_cast<const f32x4*>(s_in + sbase + (size_t)(rg + 32 * i) * kGdnD + j0) : zero4();
  for (int t = 0; t < T; ++t) {
    const int par = t & 1;
    const size_t tok = (size_t)b * T + t;
    if (t + 1 < T) rec_load(nxt, q, k, v, g, beta, tok + 1, Hk, kh, H, h, rg, j0, lane);
    // partial column sums over this thread's rows, then over the 8 row groups of the wave
    f32x4 a, c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = s[0][e] * cur.kr[0] + s[1][e] * cur.kr[1] + s[2][e] * cur.kr[2] + s[3][e] * cur.kr[3];
      c[e] = s[0][e] * cur.qr[0] + s[1][e] * cur.qr[1] + s[2][e] * cur.qr[2] + s[3][e] * cur.qr[3];
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
      red[par][wave][lane][0] = a;
      red[par][wave][lane][1] = c;
    }
    // norms of this token's q and k (every wave forms them itself)
    float sq = cur.q2[0] * cur.q2[0] + cur.q2[1] * cur.q2[1];
    float sk = cur.k2[0] * cur.k2[0] + cur.k2[1] * cur.k2[1];
    float sqk = cur.q2[0] * cur.k2[0] + cur.q2[1] * cur.k2[1];
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    sqk = wave_sum(sqk);
    lds_barrier();
    f32x4 A = red[par][0][cq][0], C = red[par][0][cq][1];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const f32x4 a2 = red[par][w][cq][0], c2 = red[par][w][cq][1];
#pragma unroll
      for (int e = 0; e < 4; ++e) { A[e] += a2[e]; C[e] += c2[e]; }
    }
    const float rk = l2norm ? rsqrtf(sk + 1e-6f) : 1.f;
    const float rqs = (l2norm ? rsqrtf(sq + 1e-6f) : 1.f) * scale;
    const float qk = sqk * rqs * rk;
    const float alpha = expf(cur.g);
    float kk[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) kk[i] = cur.kr[i] * rk;
    f32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = cur.beta * (cur.vv[e] - alpha * rk * A[e]);
      out[e] = alpha * rqs * C[e] + qk * d;
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i][e] = alpha * s[i][e] + kk[i] * d;
    }
    if (rg == 0) {
      Tin* orow = o + (tok * H + h) * kGdnD + j0;
#pragma unroll
      for (int e = 0; e < 4; ++e) orow[e] = from_f32<Tin>(out[e]);
    }
    if (t + 1 < T) cur = nxt;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<f32x4*>(s_out + sbase + (size_t)(rg + 32 * i) * kGdnD + j0) = s[i];
}

}  // namespace q35

extern "C" int q35_gdn_recurrent(const void* q, const void* k, const void* v, const float* g, const float* beta,
                                 const float* initial_state, float* final_state, void* out, int64_t B, int64_t T,
                                 int64_t Hk, int64_t H, int64_t Dk, int64_t Dv, int dtype, float scale,
                                 int use_qk_l2norm, q35_stream_t stream) {
  using namespace q35;
  if (!q || !k || !v || !g || !beta || !final_state || !out) return Q35_EINVAL;
  if (B <= 0 || T <= 0 || Hk <= 0 || H <= 0 || Dk <= 0 || Dv <= 0 || H % Hk != 0) return Q35_EINVAL;
  if (Dk != kGdnD || Dv != kGdnD) return Q35_EUNSUPPORTED;
  if (B > 65535 || H > 65535 || T > 0x7fffffff / (H > Hk ? H : Hk) / kGdnD) return Q35_EUNSUPPORTED;
  // the state is read and written as 16-byte vectors
  if (((uintptr_t)final_state & 15) || (initial_state && ((uintptr_t)initial_state & 15))) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 grid(kGdnD / kGdnJS, (unsigned)H, (unsigned)B), block(256);
  if (dtype == Q35_F32)
    hipLaunchKernelGGL(gdn_recurrent_kernel<float>, grid, block, 0, st, (const float*)q, (const float*)k,
                       (const float*)v, g, beta, initial_state, final_state, (float*)out, (int)T, (int)Hk, (int)H,
                       scale, use_qk_l2norm);
  else if (dtype == Q35_BF16)
    hipLaunchKernelGGL(gdn_recurrent_kernel<__bf16>, grid, block, 0, st, (const __bf16*)q, (const __bf16*)k,
                       (const __bf16*)v, g, beta, initial_state, final_state, (__bf16*)out, (int)T, (int)Hk, (int)H,
                       scale, use_qk_l2norm);
  else
    return Q35_EUNSUPPORTED;
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}
