// Int8 GEMM for the prefill projections: y[m, n] = sum_k x[m, k] W[n, k] s(n, k) for many rows of x (the decode
// step's few rows use gemv.hip). x fp32 [M, K], W int8 [N, K] row-major with one fp32 scale per group of 128 inputs
// of a row (s(n, k) = scale[n][k / 128], the engine's q8 format) or per output row (s(n, k) = scale[n]), y fp32.
//
// Reference: the engine's int8 `matmul` (engine/kernels.js:97-151: 64 x 64 tiles, used when M > 32; q8 weights of
// engine/kernels.js:15-47) and the MLP path with the neuron hook (`swiglu`, engine/kernels_qwen35.js:250-279).
//
// Arithmetic: bf16 MFMA (v_mfma_f32_32x32x16_bf16) with fp32 accumulation. Each x is split into hi = bf16(x) and
// lo = bf16(x - hi), so x = hi + lo up to 2^-17 |x|; the int8 weights are exact in bf16. Two products per tile
// (hi W + lo W) therefore give the fp32 product to about 1e-5 relative, which keeps the prefill on the fp32 numerics
// of the reference path (HF runs these projections in fp32). Group scales (GS): the products of one 128-input group
// accumulate into a second register set, which is added to the result scaled by the group's scale of the column.
// Epilogues: store, accumulate into y (the residual add after down_proj / out_proj), or SwiGLU over interleaved
// (gate, up) row pairs with the neuron pushes applied, writing y[m, n / 2] (fp32, or in the split layout below for
// down_proj to read without splitting).
//
// Two kernels:
//   gemm_q8_dma_kernel (N >= 2048, K <= 2048: the gate/up and input projections): 128 x 256 tiles, one block of 8
//     waves per CU, each wave a 64 x 64 output tile. x (fp32) and W (int8) go global -> LDS by DMA (global_load_lds,
//     no registers) in four stages of 32 K. What bounds this product on MI355X is VALU issue and the matrix core's
//     idle time around barriers, not bandwidth (a 64-lane VALU instruction takes 4 cycles): each stage's x is split
//     into bf16 hi / lo planes once per block (every element converted once, not once per wave that reads it), W
//     stays int8 in LDS and each wave widens only its own fragments, and there is one barrier per stage: iteration s
//     waits for stage s + 1, crosses the barrier, hands stage s's DMA buffer to stage s + 4, reads its A fragments,
//     splits stage s + 1's x while the other waves' MFMAs run, issues its MFMAs and reads stage s + 1's W fragments
//     (so that stage s's buffer is free at the next barrier). The tiles of one XCD are consecutive (n fastest inside
//     an m panel), so a panel's x stays in that XCD's L2. LDS rows are XOR-swizzled so that the 16-byte accesses of
//     16 consecutive lanes hit distinct banks. The SwiGLU epilogue splits each (gate, up) lane pair's rows between
//     the two lanes.
//   gemm_q8_rs_kernel (the rest: the N = 1024 output and down projections): 2 x 2 waves over BM x 128 tiles, x and W
//     staged through registers into LDS (split and widened on the way), the next K step's loads issued before the
//     current step's MFMAs; two blocks per CU.
// Split input (XS, q35_gemm_q8_split): x arrives already split by its producer, in the same bytes as fp32 x: each
// group of 8 consecutive inputs of a row is 32 bytes, the 8 bf16 hi parts then the 8 bf16 lo parts (the split above,
// rounded the same way). Both kernels then skip the split: the DMA kernel copies the 16-byte hi and lo pieces
// straight into the planes its A fragments are read from (no fp32 stage, no conversion pass), the register-staged
// kernel stores the loaded pieces as they are. The products, and so y, are bitwise those of the fp32 input.
// bf16 input (q35_gemm_q8_bf16, the attention output): hi = x exactly and lo = 0, so the register-staged kernel
// issues only the hi products (the skipped products are exact zeros): bitwise the product of x.float() wherever the
// fp32 input also runs the register-staged kernel (N < 2048 or K > 2048); for the wide shapes the fp32 input runs the
// DMA kernel, whose MFMAs group K differently, and the two agree to fp32 rounding.
#include <type_traits>

#include "q35_common.h"
#include "q35hip.h"

namespace q35 {

constexpr int kGN = 128;  // output columns per block (register-staged kernel)
constexpr int kGK = 64;   // K step (register-staged kernel)
constexpr int kQK = 32;   // K per pipeline stage (DMA kernel)

enum GemmEpi : int { kGemmStore = 0, kGemmAccumulate = 1, kGemmSwiglu = 2, kGemmSwigluSplit = 3 };

__device__ __forceinline__ int gsw(int r, int s) { return s ^ (r & 7); }
__device__ __forceinline__ float gemm_silu(float x) { return silu_f(x); }

// Whether any of the push records can touch neurons nlo .. nhi - 1 (a record for every neuron, or for one in the
// range): a block whose neurons no record touches skips the per-output push loop (the model passes a fixed number of
// records, unused ones matching no neuron). Uniform: the records are read with scalar loads.
__device__ __forceinline__ bool gemm_pushes_touch(const q35_push* ps, int npush, int nlo, int nhi) {
  bool any = false;
  for (int p = 0; p < npush; ++p) {
    const int pn = ps[p].neuron;
    any |= pn < 0 || (pn >= nlo && pn < nhi);
  }
  return any;
}
// the batch row of token row m (rows of T tokens each), min(m / T, 3), without a division
__device__ __forceinline__ int gemm_push_row(int m, int T) {
  return (int)(m >= T) + (int)((int64_t)m >= 2 * (int64_t)T) + (int)((int64_t)m >= 3 * (int64_t)T);
}

// y[n] of an activation row, given p = the row + gemm_act_col(n, ys): fp32, or (ys) in the split layout (n's bf16
// hi and lo parts in its group of 8)
__device__ __forceinline__ int gemm_act_col(int n, int ys) { return ys ? 8 * (n >> 3) : n; }
__device__ __forceinline__ void gemm_store_act(float* p, int n, float a, int ys) {
  if (ys) {
    __bf16* g = reinterpret_cast<__bf16*>(p);
    const bf16_hl t = bf16_split(a);
    g[n & 7] = t.hi;
    g[8 + (n & 7)] = t.lo;
  } else {
    *p = a;
  }
}

// SwiGLU activation capture (p may be NULL): the activation of neuron n of global row m goes to
// p[(m / T) ldcr + (m % T) ldc + n], fp32, whatever the layout of y
struct GemmCap {
  float* p;
  int64_t ldc, ldcr;
};
__device__ __forceinline__ void gemm_capture(const GemmCap& c, int m, int T, int n, float a) {
  if (c.p) c.p[(int64_t)(m / T) * c.ldcr + (int64_t)(m % T) * c.ldc + n] = a;
}

__device__ __forceinline__ float gemm_push(const q35_push* ps, int n, int row, float a) {
  const int pn = ps->neuron;
  if (pn != n && pn >= 0) return a;
  const float v = ps->vals[row];
  return ps->mode ? a * v : a + v;
}

// 8 consecutive fp32 values as bf16 hi and lo parts
__device__ __forceinline__ void split8(const f32x4& a, const f32x4& b, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const bf16_hl t = bf16_split(e < 4 ? a[e] : b[e - 4]);
    hi[e] = t.hi;
    lo[e] = t.lo;
  }
}
// 8 int8 values (two 32-bit words) as bf16 (exact)
__device__ __forceinline__ bf16x8 i8tobf(uint32_t w0, uint32_t w1) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t w = e < 4 ? w0 : w1;
    r[e] = (__bf16)(float)((int32_t)(w << (24 - 8 * (e & 3))) >> 24);
  }
  return r;
}

__device__ __forceinline__ uint32_t gemm_lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// 16 bytes per lane from global memory to LDS (lane i's bytes land at M0 + 16 i), from a uniform 64-bit base (moved
// to scalar registers) and a 32-bit per-lane byte offset; no registers hold the data. Inline asm, so that the
// compiler neither moves LDS accesses across it nor waits for it: completion is awaited with explicit vmcnt counts,
// and the K loop issues no other vector memory load.
__device__ __forceinline__ void gemm_dma16s(const void* sbase, uint32_t voff, uint32_t lds_dst) {
  const uint64_t a = reinterpret_cast<uint64_t>(sbase);
  const uint64_t u = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_dst), "v"(voff),
               "s"(reinterpret_cast<const void*>(u))
               : "memory", "m0");
}
template <int N> __device__ __forceinline__ void gemm_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// ---------------------------------------------------------------------------------------------------------------
// DMA kernel: 128 x 256 tiles, 512 threads (wave w: rows 64 (w / 4), columns 64 (w % 4)), four DMA stages.
constexpr int kDBM = 128, kDBN = 256, kDNS = 4;
constexpr int kDGS = 16;               // groups of 128 inputs whose scales the block holds (K <= 2048)
// LDS layouts (a 16-byte access by 16 consecutive lanes is conflict-free when the 16 addresses fall in distinct
// 16-byte slots of a 256-byte window; the swizzles below are chosen for the patterns that read each area):
constexpr int kDXB = kDBM * kQK * 4;   // x bytes per stage: fp32 rows of 128 B, 16-byte chunk c at c ^ ((row >> 1) & 1)
constexpr int kDWB = kDBN * kQK;       // W bytes per stage: int8 rows of 32 B, 16-byte half h at h ^ ((row >> 3) & 1)
constexpr int kDSB = kDXB + kDWB;
constexpr int kDXC = kDBM * kQK * 2;   // one bf16 plane (hi or lo) of a stage's x: rows of 64 B, 16-byte chunk c at
                                       // c ^ ((row >> 2) & 3)
// DMA instructions (1 KB) per wave and stage: two of x (rows 8 q .. 8 q + 7, q = w, w + 8) and one of W (rows
// 32 w .. 32 w + 31)

template <int EPI, bool GS, bool XS>
__global__ __launch_bounds__(512, 1) void gemm_q8_dma_kernel(const float* __restrict__ X, int64_t ldx,
                                                             const int8_t* __restrict__ W,
                                                             const float* __restrict__ ws, float* __restrict__ Y,
                                                             int64_t ldy, int M, int N, int K,
                                                             const q35_push* __restrict__ pushes, int npush, int T,
                                                             int moff, int ys, GemmCap cap) {
  __shared__ __attribute__((aligned(16))) char smem[kDNS * kDSB];
  __shared__ __attribute__((aligned(16))) char xc[XS ? 1 : 2][2][XS ? 16 : kDXC];  // [buffer][hi, lo] (fp32 x)
  __shared__ float gscale[GS ? kDGS * kDBN : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // wave w owns rows 64 (w / 4) .. + 63 and columns 64 (w % 4) .. + 63: 2 x 2 MFMA tiles of 32 x 32
  constexpr int MT = 2, NT = 2;
  const int wm = wv >> 2, wn = wv & 3;
  const int l32 = lane & 31, lh = lane >> 5;
  // tile order: block b runs on XCD b % 8, which gets ceil((ntiles - j) / 8) blocks; XCD j takes that many
  // consecutive tiles from j q + min(j, r) (ntiles = 8 q + r), n fastest inside an m panel
  const int nbn = (N + kDBN - 1) / kDBN;
  const int ntiles = nbn * ((M + kDBM - 1) / kDBM);
  const int xj = (int)(blockIdx.x & 7), xq = ntiles >> 3, xr = ntiles & 7;
  const int tile = xj * xq + min(xj, xr) + (int)(blockIdx.x >> 3);
  const int bm = tile / nbn, bn = tile - bm * nbn;
  const int m0 = bm * kDBM, n0 = bn * kDBN;
  const int G = K >> 7;
  const int KT = K / kQK;

  // DMA sources of this lane (32-bit byte offsets from x and W; the launcher keeps both under 4 GB)
  uint32_t xsrc[2], xoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if constexpr (XS) {
      // split x: instruction i fills rows 16 w .. 16 w + 15 of the stage's plane i (hi, lo), laid out as the fp32
      // path's converted planes; lane -> row 16 w + lane / 4, slot lane % 4 of the row, which holds the group of 8
      // inputs c = slot ^ ((row >> 2) & 3) (the group's 16 bytes of plane i)
      const int row = 16 * wv + (lane >> 2);
      const int c = (lane & 3) ^ ((row >> 2) & 3);
      xsrc[i] = (uint32_t)(((size_t)min(m0 + row, M - 1) * ldx + 8 * c) * 4 + 16 * i);
      xoff[i] = (uint32_t)(i * kDXC + wv * 1024);
    } else {
      const int q = wv + 8 * i;
      const int row = 8 * q + (lane >> 3);
      const int c = (lane & 7) ^ ((row >> 1) & 1);
      xsrc[i] = (uint32_t)(((size_t)min(m0 + row, M - 1) * ldx + 4 * c) * 4);
      xoff[i] = (uint32_t)(q * 1024);
    }
  }
  uint32_t wsrc, woff;
  {
    const int row = 32 * wv + (lane >> 1);
    const int h = (lane & 1) ^ ((row >> 3) & 1);
    wsrc = (uint32_t)((size_t)min(n0 + row, N - 1) * K + 16 * h);
    woff = (uint32_t)(kDXB + wv * 1024);
  }
  const uint32_t lds0 = gemm_lds_u32(smem);
  auto issue = [&](int s, int buf) {
    const uint32_t base = lds0 + buf * kDSB;
    gemm_dma16s(X, xsrc[0] + (uint32_t)(s * kQK * 4), base + xoff[0]);
    gemm_dma16s(X, xsrc[1] + (uint32_t)(s * kQK * 4), base + xoff[1]);
    gemm_dma16s(W, wsrc + (uint32_t)(s * kQK), base + woff);
  };
  auto wait_stage = [&](int s) {  // stage s has landed in every wave's part; every wave is past its earlier reads
    const int ahead = min(KT - 1 - s, kDNS - 2);  // stages issued after s that may still be in flight
    if (ahead >= 2) gemm_wait_vm<6>();
    else if (ahead == 1) gemm_wait_vm<3>();
    else gemm_wait_vm<0>();
    lds_barrier();
  };
  // the split of a stage's x: thread -> row tid / 4, k 8 (tid % 4) .. + 7
  const int cr = tid >> 2, c8 = tid & 3;
  const uint32_t cv0 = (uint32_t)(cr * 128 + (((2 * c8) ^ ((cr >> 1) & 1)) << 4));
  const uint32_t cv1 = (uint32_t)(cr * 128 + (((2 * c8 + 1) ^ ((cr >> 1) & 1)) << 4));
  const uint32_t cvw = (uint32_t)(cr * 64 + ((c8 ^ ((cr >> 2) & 3)) << 4));
  auto convert = [&](int s, int xb) {
    const char* st = smem + (s % kDNS) * kDSB;
    bf16x8 hi, lo;
    split8(*reinterpret_cast<const f32x4*>(st + cv0), *reinterpret_cast<const f32x4*>(st + cv1), hi, lo);
    *reinterpret_cast<bf16x8*>(xc[xb][0] + cvw) = hi;
    *reinterpret_cast<bf16x8*>(xc[xb][1] + cvw) = lo;
  };
  // fragment offsets: A rows 64 wm + 32 mt + l32 in the bf16 planes, chunk 2 lh + j (k = 16 lh + 8 j .. + 7); B rows
  // 64 wn + 32 nt + l32 of the stage's W, half lh (k = 16 lh .. + 15: fragment j is its bytes 8 j .. 8 j + 7). Rows
  // 32 apart have the same swizzle (A offsets step by 2048, B offsets by 1024).
  uint32_t aoff[2];
  {
    const int r = wm * 64 + l32;
#pragma unroll
    for (int j = 0; j < 2; ++j) aoff[j] = (uint32_t)(r * 64 + (((2 * lh + j) ^ ((r >> 2) & 3)) << 4));
  }
  const uint32_t boff = (uint32_t)(kDXB + (wn * 64 + l32) * 32 + ((lh ^ ((l32 >> 3) & 1)) << 4));
  // A fragments of one stage: from the converted planes (fp32 x, read at the start of the stage's iteration) or,
  // for split x, from the stage's DMA buffer (read at the end of the previous iteration, like W, so that the buffer
  // is free for the stage issued after the next barrier)
  bf16x8 ah[2][MT], al[2][MT];
  auto read_a = [&](const char* xh, const char* xl) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        ah[j][mt] = *reinterpret_cast<const bf16x8*>(xh + aoff[j] + mt * 2048);
        al[j][mt] = *reinterpret_cast<const bf16x8*>(xl + aoff[j] + mt * 2048);
      }
  };
  auto read_a_stage = [&](int s) {
    const char* st = smem + (s % kDNS) * kDSB;
    read_a(st, st + kDXC);
  };

  f32x16 acc[MT][NT], gacc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      acc[mt][nt] = zero16();
      gacc[mt][nt] = zero16();  // (overwritten: a group's first MFMAs start from zero)
    }

#pragma unroll
  for (int s = 0; s < kDNS - 1; ++s)
    if (s < KT) issue(s, s);
  if constexpr (GS) {
    // the block's group scales, [group][column]: loaded behind the first stages (the wait for them ends about when
    // stage 0 lands, which the loop waits for anyway), so that no register load waits inside the K loop
    for (int i = tid; i < G * kDBN; i += 512) {
      const int g = i / kDBN, c = i - g * kDBN;
      gscale[i] = ws[(size_t)min(n0 + c, N - 1) * G + g];
    }
  }
  // one barrier per stage. Iteration s: wait for stage s + 1 and cross the barrier (after it: stage s's split is
  // complete, every wave has read stage s's W and is done with the other x buffer); hand stage s's DMA buffer to
  // stage s + 4; read stage s's A fragments; split stage s + 1's x (its VALU work overlaps the other waves' MFMAs);
  // issue stage s's MFMAs; read stage s + 1's W fragments for the next iteration.
  u32x4 wr[NT];
  auto read_w = [&](int s) {
    const char* st = smem + (s % kDNS) * kDSB;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) wr[nt] = *reinterpret_cast<const u32x4*>(st + boff + nt * 1024);
  };
  wait_stage(0);
  if (kDNS - 1 < KT) issue(kDNS - 1, kDNS - 1);
  if constexpr (XS) read_a_stage(0);
  else convert(0, 0);
  read_w(0);

  auto stage = [&](int s, auto ph_c) {
    constexpr int ph = decltype(ph_c)::value;
    if (s + 1 < KT) wait_stage(s + 1);
    else lds_barrier();
    if (s + kDNS < KT) issue(s + kDNS, s % kDNS);
    if constexpr (!XS) {
      read_a(xc[s & 1][0], xc[s & 1][1]);
      if (s + 1 < KT) convert(s + 1, (s + 1) & 1);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf16x8 b[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) b[nt] = i8tobf(wr[nt][2 * j], wr[nt][2 * j + 1]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          if constexpr (GS) gacc[mt][nt] = mfma32(ah[j][mt], b[nt], (ph == 0 && j == 0) ? zero16() : gacc[mt][nt]);
          else acc[mt][nt] = mfma32(ah[j][mt], b[nt], acc[mt][nt]);
        }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          f32x16& d = GS ? gacc[mt][nt] : acc[mt][nt];
          d = mfma32(al[j][mt], b[nt], d);
        }
    }
    if (s + 1 < KT) {
      read_w(s + 1);
      if constexpr (XS) read_a_stage(s + 1);
    }
    if constexpr (GS && ph == 3) {  // end of a group of 128 inputs: fold it in with its scale
      const int g = s >> 2;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float sc = gscale[g * kDBN + wn * 64 + 32 * nt + l32];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[mt][nt][r] += sc * gacc[mt][nt][r];
      }
    }
  };
  if constexpr (GS) {
    for (int s = 0; s < KT; s += 4) {  // K is a multiple of 128
      stage(s, std::integral_constant<int, 0>{});
      stage(s + 1, std::integral_constant<int, 1>{});
      stage(s + 2, std::integral_constant<int, 2>{});
      stage(s + 3, std::integral_constant<int, 3>{});
    }
  } else {
    for (int s = 0; s < KT; ++s) stage(s, std::integral_constant<int, 0>{});
  }

  // epilogue: lane holds column n = n0 + 64 wn + 32 nt + l32, rows m0 + 64 wm + 32 mt + 8 (r / 4) + 4 lh + r % 4
  const int mb = m0 + wm * 64 + 4 * lh;
  const bool pushes_here = EPI == kGemmSwiglu && gemm_pushes_touch(pushes, npush, n0 >> 1, (n0 + kDBN) >> 1);
  int64_t roff[16];  // element offsets of a tile's 16 accumulator rows from its first (uniform): one add per output
#pragma unroll
  for (int r = 0; r < 16; ++r) roff[r] = (int64_t)(8 * (r >> 2) + (r & 3)) * ldy;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = n0 + wn * 64 + 32 * nt + l32;
    const float sc = GS ? 1.f : ws[min(n, N - 1)];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float* yt = Y + (int64_t)(mb + 32 * mt) * ldy;
      float* ytn = yt + (EPI == kGemmSwiglu ? gemm_act_col(n >> 1, ys) : n);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mb + 32 * mt + 8 * (r >> 2) + (r & 3);
        const float v = acc[mt][nt][r] * sc;
        if (EPI == kGemmSwiglu) {
          // columns n (gate, even lane) and n + 1 (up, odd lane) of a neuron: the even lane finishes the rows with
          // r < 8, the odd lane those with r >= 8
          const float o = __shfl_xor(v, 1, 64);
          const bool odd = (l32 & 1) != 0;
          if (odd == (r >= 8) && m < M && (n | 1) < N) {
            const int neuron = n >> 1;
            const float gate = odd ? o : v, up = odd ? v : o;
            float a = gemm_silu(gate) * up;
            if (pushes_here) {
              const int row = gemm_push_row(moff + m, T);
              for (int p = 0; p < npush; ++p) a = gemm_push(pushes + p, neuron, row, a);
            }
            gemm_store_act(ytn + roff[r], neuron, a, ys);
            gemm_capture(cap, moff + m, T, neuron, a);
          }
        } else if (m < M && n < N) {
          float* dst = ytn + roff[r];
          *dst = EPI == kGemmAccumulate ? *dst + v : v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Register-staged kernel: 2 x 2 waves over BM x 128 tiles (BM 64 or 128), K in steps of 64. Per K step the block
// stages x[BM, 64] (split into hi and lo) and W[128, 64] (int8 -> bf16) in LDS, rows of 64 bf16 = 8 segments of 16
// bytes, segment s of row r at s ^ (r & 7). The next step's global loads are issued before the current step's MFMAs,
// so they are in flight during them. Blocks run n-fastest inside an m panel.
// XF: x fp32 (0), in the split layout (1), or bf16 (2: hi = x exactly, lo = 0, so the lo products are skipped)
template <int BM, int EPI, bool GS, int XF>
__global__ __launch_bounds__(256, 2) void gemm_q8_rs_kernel(const float* __restrict__ X, int64_t ldx,
                                                         const int8_t* __restrict__ W, const float* __restrict__ ws,
                                                         float* __restrict__ Y, int64_t ldy, int M, int N, int K,
                                                         const q35_push* __restrict__ pushes, int npush, int T,
                                                         int moff, int ys, GemmCap cap) {
  static_assert(BM == 64 || BM == 128, "rows per block");
  constexpr int MT = BM / 64;         // 32-row MFMA tiles per wave along M (a wave covers BM / 2 rows)
  constexpr int TPR = 256 / BM;       // threads per staged row of x
  constexpr int SPT = 8 / TPR;        // 16-byte segments (8 k values) of x per thread
  __shared__ __attribute__((aligned(16))) bf16x8 Ah[BM * 8];
  __shared__ __attribute__((aligned(16))) bf16x8 Al[BM * 8];
  __shared__ __attribute__((aligned(16))) bf16x8 Bs[kGN * 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int nbn = (N + kGN - 1) / kGN;
  const int bm = blockIdx.x / nbn, bn = blockIdx.x - bm * nbn;
  const int m0 = bm * BM, n0 = bn * kGN;

  // staging assignment: x row ar, segments as0 .. as0 + SPT - 1; W row br, segments 4 bh .. 4 bh + 3
  const int ar = tid / TPR, as0 = (tid % TPR) * SPT;
  const int br = tid >> 1, bh = tid & 1;
  const bool av = m0 + ar < M, bv = n0 + br < N;
  // (bf16 x: element offsets count 2-byte values; xa[s][0] then holds the segment's 8 values)
  const float* xrow = XF == 2 ? reinterpret_cast<const float*>(reinterpret_cast<const __bf16*>(X) +
                                                               (size_t)min(m0 + ar, M - 1) * ldx + 8 * as0)
                              : X + (size_t)min(m0 + ar, M - 1) * ldx + 8 * as0;
  const int8_t* wrow = W + (size_t)min(n0 + br, N - 1) * K + 32 * bh;

  f32x4 xa[SPT][2];
  u32x4 wb[2];
  auto load = [&](int k0) {
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      if constexpr (XF == 2) {
        xa[s][0] = *reinterpret_cast<const f32x4*>(xrow + (k0 + 8 * s) / 2);
      } else {
        xa[s][0] = *reinterpret_cast<const f32x4*>(xrow + k0 + 8 * s);
        xa[s][1] = *reinterpret_cast<const f32x4*>(xrow + k0 + 8 * s + 4);
      }
    }
    wb[0] = *reinterpret_cast<const u32x4*>(wrow + k0);
    wb[1] = *reinterpret_cast<const u32x4*>(wrow + k0 + 16);
  };
  auto stage = [&]() {
    const bf16x8 z = {};
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      bf16x8 hi, lo;
      if constexpr (XF == 1) {  // split x: the group's 16 bytes of hi parts, then its 16 bytes of lo parts
        hi = __builtin_bit_cast(bf16x8, xa[s][0]);
        lo = __builtin_bit_cast(bf16x8, xa[s][1]);
      } else if constexpr (XF == 2) {
        hi = __builtin_bit_cast(bf16x8, xa[s][0]);
      } else {
        split8(xa[s][0], xa[s][1], hi, lo);
      }
      const int idx = ar * 8 + gsw(ar, as0 + s);
      Ah[idx] = av ? hi : z;
      if constexpr (XF != 2) Al[idx] = av ? lo : z;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4& w = wb[j >> 1];
      const bf16x8 b = i8tobf(w[2 * (j & 1)], w[2 * (j & 1) + 1]);
      Bs[br * 8 + gsw(br, 4 * bh + j)] = bv ? b : z;
    }
  };

  f32x16 acc[MT][2], gacc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      acc[mt][nt] = zero16();
      gacc[mt][nt] = zero16();
    }

  const int l32 = lane & 31, lh = lane >> 5;
  // GS: the lane's two columns' scale rows (column n = n0 + wn 64 + 32 nt + l32)
  const float* srow[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) srow[nt] = ws + (size_t)min(n0 + wn * 64 + 32 * nt + l32, N - 1) * (K >> 7);
  float gsc[2] = {0.f, 0.f};
  load(0);
  for (int k0 = 0; k0 < K; k0 += kGK) {
    __syncthreads();  // every wave is done reading the previous step's tiles
    stage();
    if (k0 + kGK < K) load(k0 + kGK);  // next step's loads fly during this step's MFMAs
    if (GS && (k0 & 127) == 0) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) gsc[nt] = srow[nt][k0 >> 7];
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int sg = 2 * kk + lh;
      bf16x8 ah[MT], al[MT], b[2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int r = wm * (BM / 2) + 32 * mt + l32;
        ah[mt] = Ah[r * 8 + gsw(r, sg)];
        if constexpr (XF != 2) al[mt] = Al[r * 8 + gsw(r, sg)];
      }
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int r = wn * 64 + 32 * nt + l32;
        b[nt] = Bs[r * 8 + gsw(r, sg)];
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          f32x16& d = GS ? gacc[mt][nt] : acc[mt][nt];
          d = mfma32(ah[mt], b[nt], d);
          if constexpr (XF != 2) d = mfma32(al[mt], b[nt], d);
        }
    }
    if (GS && ((k0 + kGK) & 127) == 0) {  // end of a group: fold it in with its scale
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[mt][nt][r] += gsc[nt] * gacc[mt][nt][r];
          gacc[mt][nt] = zero16();
        }
    }
  }

  // epilogue: lane holds column n = n0 + wn 64 + 32 nt + l32, rows m0 + wm BM/2 + 32 mt + 8 (r / 4) + 4 lh + r % 4
  const bool pushes_here = EPI == kGemmSwiglu && gemm_pushes_touch(pushes, npush, n0 >> 1, (n0 + kGN) >> 1);
  int64_t roff[16];  // element offsets of a tile's 16 accumulator rows from its first (uniform): one add per output
#pragma unroll
  for (int r = 0; r < 16; ++r) roff[r] = (int64_t)(8 * (r >> 2) + (r & 3)) * ldy;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int n = n0 + wn * 64 + 32 * nt + l32;
    const float s = GS ? 1.f : ws[min(n, N - 1)];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int mt0 = m0 + wm * (BM / 2) + 32 * mt + 4 * lh;
      float* ytn = Y + (int64_t)mt0 * ldy + (EPI == kGemmSwiglu ? gemm_act_col(n >> 1, ys) : n);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mt0 + 8 * (r >> 2) + (r & 3);
        const float v = acc[mt][nt][r] * s;
        if (EPI == kGemmSwiglu) {
          const float up = __shfl_xor(v, 1, 64);  // the odd column of the pair sits in the neighbouring lane
          if ((l32 & 1) == 0 && m < M && n + 1 < N) {
            const int neuron = n >> 1;
            float a = gemm_silu(v) * up;
            if (pushes_here) {
              const int row = gemm_push_row(moff + m, T);
              for (int p = 0; p < npush; ++p) a = gemm_push(pushes + p, neuron, row, a);
            }
            gemm_store_act(ytn + roff[r], neuron, a, ys);
            gemm_capture(cap, moff + m, T, neuron, a);
          }
        } else if (m < M && n < N) {
          float* dst = ytn + roff[r];
          *dst = EPI == kGemmAccumulate ? *dst + v : v;
        }
      }
    }
  }
}

}  // namespace q35

namespace q35 {

template <int XF>
static int gemm_rs_launch(const float* x, int64_t ldx, const int8_t* W, const float* w_scale, float* y, int64_t ldy,
                          int64_t M, int64_t N, int64_t K, int epilogue, bool gs, const q35_push* pushes, int64_t npush,
                          int64_t T, int64_t moff, int ys, const GemmCap& cap, hipStream_t st) {
  const int64_t nbn = (N + kGN - 1) / kGN;
  // 128-row tiles when they still give at least two blocks per compute unit, else 64-row tiles
  const bool big = ((M + 127) / 128) * nbn >= 512;
  const int BM = big ? 128 : 64;
  const int64_t nblocks = ((M + BM - 1) / BM) * nbn;
  if (nblocks > 0x7fffffff) return Q35_EUNSUPPORTED;
#define Q35_GEMM_LAUNCH(BMV, E, G)                                                                                   \
  hipLaunchKernelGGL((gemm_q8_rs_kernel<BMV, E, G, XF>), dim3((unsigned)nblocks), dim3(256), 0, st, x, ldx, W,       \
                     w_scale, y, ldy, (int)M, (int)N, (int)K, pushes, (int)npush, (int)T, (int)moff, ys, cap)
#define Q35_GEMM_EPI(BMV, G)                                              \
  if (epilogue == kGemmStore) Q35_GEMM_LAUNCH(BMV, kGemmStore, G);        \
  else if (epilogue == kGemmAccumulate) Q35_GEMM_LAUNCH(BMV, kGemmAccumulate, G); \
  else Q35_GEMM_LAUNCH(BMV, kGemmSwiglu, G);
  if (big) {
    if (gs) { Q35_GEMM_EPI(128, true) } else { Q35_GEMM_EPI(128, false) }
  } else {
    if (gs) { Q35_GEMM_EPI(64, true) } else { Q35_GEMM_EPI(64, false) }
  }
#undef Q35_GEMM_EPI
#undef Q35_GEMM_LAUNCH
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

template <bool XS>
static int gemm_dma_launch(const float* x, int64_t ldx, const int8_t* W, const float* w_scale, float* y, int64_t ldy,
                           int64_t M, int64_t N, int64_t K, int epilogue, bool gs, const q35_push* pushes,
                           int64_t npush, int64_t T, int ys, const GemmCap& cap, hipStream_t st) {
  const int moff = 0;
  const int64_t nblocks = ((M + kDBM - 1) / kDBM) * ((N + kDBN - 1) / kDBN);
  if (nblocks > 0x7fffffff) return Q35_EUNSUPPORTED;
#define Q35_GEMM_DMA(E, G_)                                                                                       \
  hipLaunchKernelGGL((gemm_q8_dma_kernel<E, G_, XS>), dim3((unsigned)nblocks), dim3(512), 0, st, x, ldx, W,        \
                     w_scale, y, ldy, (int)M, (int)N, (int)K, pushes, (int)npush, (int)T, moff, ys, cap)
  if (gs) {
    if (epilogue == kGemmStore) Q35_GEMM_DMA(kGemmStore, true);
    else if (epilogue == kGemmAccumulate) Q35_GEMM_DMA(kGemmAccumulate, true);
    else Q35_GEMM_DMA(kGemmSwiglu, true);
  } else {
    if (epilogue == kGemmStore) Q35_GEMM_DMA(kGemmStore, false);
    else if (epilogue == kGemmAccumulate) Q35_GEMM_DMA(kGemmAccumulate, false);
    else Q35_GEMM_DMA(kGemmSwiglu, false);
  }
#undef Q35_GEMM_DMA
  return hipGetLastError() == hipSuccess ? Q35_OK : Q35_ELAUNCH;
}

// compute units of the current device (the DMA kernel runs one block per CU)
static int64_t gemm_cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

}  // namespace q35

namespace q35 {

// x: fp32 rows, or for XS rows in the split layout (the same bytes and leading dimension as fp32 rows)
template <bool XS, bool XB = false>
static int gemm_q8_run(const float* x, int64_t ldx, const int8_t* W, int w_dtype, const float* w_scale, float* y,
                       int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes,
                       int64_t npush, int64_t T, float* cap_p, int64_t ld_cap, int64_t ld_cap_row,
                       q35_stream_t stream) {
  if (!x || !W || !w_scale || !y || M <= 0 || N <= 0 || K <= 0 || T <= 0) return Q35_EINVAL;
  if (cap_p && (epilogue < kGemmSwiglu || ld_cap < N / 2 || ld_cap_row < N / 2 || ((uintptr_t)cap_p & 3)))
    return Q35_EINVAL;
  const GemmCap cap = {cap_p, ld_cap, ld_cap_row};
  if (w_dtype != Q35_I8 && w_dtype != Q35_I8_G128) return Q35_EUNSUPPORTED;
  const bool gs = w_dtype == Q35_I8_G128;
  if (gs && K % 128 != 0) return Q35_EUNSUPPORTED;
  if (epilogue < kGemmStore || epilogue > kGemmSwigluSplit) return Q35_EINVAL;
  // epilogue 3: SwiGLU with y in the split layout (the next product's input, read without splitting)
  const int ys = epilogue == kGemmSwigluSplit;
  if (ys) {
    epilogue = kGemmSwiglu;
    if ((N / 2) % 8 != 0 || ldy % 4 != 0 || ((uintptr_t)y & 15)) return Q35_EUNSUPPORTED;
  }
  if (npush < 0 || (npush > 0 && !pushes) || npush > 64) return Q35_EINVAL;
  if (epilogue == kGemmSwiglu ? (N % 2 != 0 || ldy < N / 2) : ldy < N) return Q35_EINVAL;
  if (ldx < K) return Q35_EINVAL;
  if (K % kGK != 0 || ldx % (XB ? 8 : 4) != 0 || ((uintptr_t)x & 15) || ((uintptr_t)W & 15)) return Q35_EUNSUPPORTED;
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return Q35_EUNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // bf16 x: the register-staged kernel (one product per tile: the lo parts are zero)
  if constexpr (XB)
    return gemm_rs_launch<2>(x, ldx, W, w_scale, y, ldy, M, N, K, epilogue, gs, pushes, npush, T, 0, ys, cap, st);
  // wide products with K <= 2048 (and x, W addressable with 32-bit byte offsets): the DMA kernel
  if (N >= 2048 && K <= 128 * kDGS && ((M - 1) * ldx + K) * 4 <= 0xffffffffLL && N * K <= 0xffffffffLL) {
    // One block per CU, so a last round of blocks that is mostly empty costs as much as a full one. A partial last
    // column tile that costs a whole extra round (the GDN input projection: 8192 + 32 columns) runs on the
    // register-staged kernel after the full tiles (store and accumulate epilogues: their columns are independent);
    // when the last round is less than half full, the rows past the m panels that fill one round fewer run on the
    // register-staged kernel too (gate/up: 1,344 tiles, 5.25 rounds -> 45 m panels on the DMA kernel, 384 rows).
    const int64_t cus = gemm_cu_count();
    const int64_t mt = (M + kDBM - 1) / kDBM;
    int64_t Nd = N, Md = M;
    const int64_t nfull = N / kDBN * kDBN;
    if (epilogue != kGemmSwiglu && nfull > 0 && nfull < N) {
      const int64_t rounds_all = (mt * (N / kDBN + 1) + cus - 1) / cus, rounds_full = (mt * (N / kDBN) + cus - 1) / cus;
      if (rounds_full < rounds_all) Nd = nfull;
    }
    {
      const int64_t nbd = (Nd + kDBN - 1) / kDBN, tiles = mt * nbd, R = (tiles + cus - 1) / cus;
      if (R >= 2 && 2 * (tiles - (R - 1) * cus) < cus) {
        const int64_t M1 = ((R - 1) * cus / nbd) * kDBM;
        if (M1 > 0 && M1 < M) Md = M1;
      }
    }
    int r = gemm_dma_launch<XS>(x, ldx, W, w_scale, y, ldy, Md, Nd, K, epilogue, gs, pushes, npush, T, ys, cap, st);
    if (r != Q35_OK) return r;
    if (Md < M) {
      r = gemm_rs_launch<(XS ? 1 : 0)>(x + Md * ldx, ldx, W, w_scale, y + Md * ldy, ldy, M - Md, Nd, K, epilogue, gs,
                                       pushes, npush, T, Md, ys, cap, st);
      if (r != Q35_OK) return r;
    }
    if (Nd < N)
      r = gemm_rs_launch<(XS ? 1 : 0)>(x, ldx, W + Nd * K, w_scale + (gs ? Nd * (K / 128) : Nd), y + Nd, ldy, M,
                                       N - Nd, K, epilogue, gs, pushes, npush, T, 0, ys, cap, st);
    return r;
  }
  return gemm_rs_launch<(XS ? 1 : 0)>(x, ldx, W, w_scale, y, ldy, M, N, K, epilogue, gs, pushes, npush, T, 0, ys, cap,
                                      st);
}

}  // namespace q35

extern "C" int q35_gemm_q8(const float* x, int64_t ldx, const int8_t* W, int w_dtype, const float* w_scale,
                           float* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue,
                           const q35_push* pushes, int64_t npush, int64_t T, float* cap, int64_t ld_cap,
                           int64_t ld_cap_row, q35_stream_t stream) {
  return q35::gemm_q8_run<false>(x, ldx, W, w_dtype, w_scale, y, ldy, M, N, K, epilogue, pushes, npush, T, cap, ld_cap,
                                 ld_cap_row, stream);
}

extern "C" int q35_gemm_q8_split(const void* xs, int64_t ldx, const int8_t* W, int w_dtype, const float* w_scale,
                                 float* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue,
                                 const q35_push* pushes, int64_t npush, int64_t T, float* cap, int64_t ld_cap,
                                 int64_t ld_cap_row, q35_stream_t stream) {
  return q35::gemm_q8_run<true>(static_cast<const float*>(xs), ldx, W, w_dtype, w_scale, y, ldy, M, N, K, epilogue,
                                pushes, npush, T, cap, ld_cap, ld_cap_row, stream);
}

extern "C" int q35_gemm_q8_bf16(const void* xb, int64_t ldx, const int8_t* W, int w_dtype, const float* w_scale,
                                float* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue,
                                const q35_push* pushes, int64_t npush, int64_t T, float* cap, int64_t ld_cap,
                                int64_t ld_cap_row, q35_stream_t stream) {
  return q35::gemm_q8_run<false, true>(static_cast<const float*>(xb), ldx, W, w_dtype, w_scale, y, ldy, M, N, K,
                                       epilogue, pushes, npush, T, cap, ld_cap, ld_cap_row, stream);
}
