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
// which is the same arithmetic regrouped (both dot products come from one pass over the state tile).
//
// Decomposition: one block per (slice of 16 value columns, head, batch row) -> Dv/16 * H * B blocks of 256 threads.
// Thread t owns a float4 of columns (t % 4) in rows t/4 and t/4 + 64, so every wave reads 16 full 64-byte row
// segments per load. The column reductions run as xor-shuffles over lanes with equal t % 4, then across the four
// waves through LDS. Memory per launch: S read + written once (2 * 4 * Dk * Dv bytes per (b, h)).
#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kGdnD = 128;   // Dk = Dv
constexpr int kGdnJS = 16;   // value columns per block

template <typename Tin>
__global__ __launch_bounds__(256) void gdn_recurrent_kernel(const Tin* __restrict__ q, const Tin* __restrict__ k,
                                                            const Tin* __restrict__ v, const float* __restrict__ g,
                                                            const float* __restrict__ beta, const float* s_in,
                                                            float* s_out, Tin* __restrict__ o, int T, int Hk, int H,
                                                            float scale, int l2norm) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int cq = tid & 3;   // column quad of this thread
  const int r0 = tid >> 2;  // rows r0 and r0 + 64
  const int j0 = blockIdx.x * kGdnJS + cq * 4;
  const int h = blockIdx.y, b = blockIdx.z;
  const int kh = h / (H / Hk);

  __shared__ float qs[2][kGdnD], ks[2][kGdnD];
  __shared__ float red1[2][4][4];   // [parity][wave][sum q^2, sum k^2, sum q k, pad]
  __shared__ f32x4 red2[2][4][4][2];  // [parity][wave][column quad][S^T k | S^T q]

  const size_t sbase = ((size_t)b * H + h) * kGdnD * kGdnD;
  f32x4 s[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    if (s_in)
      s[p] = *reinterpret_cast<const f32x4*>(s_in + sbase + (size_t)(r0 + 64 * p) * kGdnD + j0);
    else
      s[p] = zero4();
  }

  for (int t = 0; t < T; ++t) {
    const int par = t & 1;
    const size_t tok = (size_t)b * T + t;
    // per-token scalars and this thread's value columns, issued first so they overlap the reductions
    const float alpha = expf(g[tok * H + h]);
    const float be = beta[tok * H + h];
    const Tin* vrow = v + (tok * H + h) * kGdnD + j0;
    float vv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) vv[e] = to_f32(vrow[e]);
    float qv = 0.f, kv = 0.f;
    if (tid < kGdnD) {
      qv = to_f32(q[(tok * Hk + kh) * kGdnD + tid]);
      kv = to_f32(k[(tok * Hk + kh) * kGdnD + tid]);
      qs[par][tid] = qv;
      ks[par][tid] = kv;
    }
    float sq = qv * qv, sk = kv * kv, sqk = qv * kv;
    if (wave < 2) {  // waves 2 and 3 hold no q/k elements
      sq = wave_sum(sq);
      sk = wave_sum(sk);
      sqk = wave_sum(sqk);
      if (lane == 0) {
        red1[par][wave][0] = sq;
        red1[par][wave][1] = sk;
        red1[par][wave][2] = sqk;
      }
    }
    __syncthreads();
    const float Sq = red1[par][0][0] + red1[par][1][0];
    const float Sk = red1[par][0][1] + red1[par][1][1];
    const float Sqk = red1[par][0][2] + red1[par][1][2];
    const float rq = l2norm ? rsqrtf(Sq + 1e-6f) : 1.f;
    const float rk = l2norm ? rsqrtf(Sk + 1e-6f) : 1.f;
    const float qsc = rq * scale;
    const float qk = Sqk * rq * rk * scale;
    const float kk0 = ks[par][r0] * rk, kk1 = ks[par][r0 + 64] * rk;
    const float qq0 = qs[par][r0] * qsc, qq1 = qs[par][r0 + 64] * qsc;

    f32x4 a, c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = s[0][e] * kk0 + s[1][e] * kk1;
      c[e] = s[0][e] * qq0 + s[1][e] * qq1;
    }
#pragma unroll
    for (int off = 4; off < 64; off <<= 1) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[e] += __shfl_xor(a[e], off, 64);
        c[e] += __shfl_xor(c[e], off, 64);
      }
    }
    if (lane < 4) {
      red2[par][wave][lane][0] = a;
      red2[par][wave][lane][1] = c;
    }
    __syncthreads();
    f32x4 A = red2[par][0][cq][0], C = red2[par][0][cq][1];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const f32x4 a2 = red2[par][w][cq][0], c2 = red2[par][w][cq][1];
#pragma unroll
      for (int e = 0; e < 4; ++e) { A[e] += a2[e]; C[e] += c2[e]; }
    }
    f32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = be * (vv[e] - alpha * A[e]);
      out[e] = alpha * C[e] + qk * d;
      s[0][e] = alpha * s[0][e] + kk0 * d;
      s[1][e] = alpha * s[1][e] + kk1 * d;
    }
    if (r0 == 0) {
      Tin* orow = o + (tok * H + h) * kGdnD + j0;
#pragma unroll
      for (int e = 0; e < 4; ++e) orow[e] = from_f32<Tin>(out[e]);
    }
  }
#pragma unroll
  for (int p = 0; p < 2; ++p)
    *reinterpret_cast<f32x4*>(s_out + sbase + (size_t)(r0 + 64 * p) * kGdnD + j0) = s[p];
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
