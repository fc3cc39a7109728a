// Shared device helpers for the Qwen3.5 hybrid-attention kernels (gfx950 / CDNA4, wave64).
//
// MFMA operand layouts used throughout (v_mfma_f32_16x16x32_bf16 and v_mfma_f32_32x32x16_bf16, gfx950):
//   16x16x32:  A[16x32]  lane l holds row l%16, k = 8*(l/16) + j (j = 0..7)
//              B[32x16]  lane l holds col l%16, k = 8*(l/16) + j
//              D[16x16]  lane l holds col l%16, rows 4*(l/16) + r (r = 0..3)
//   32x32x16:  A[32x16]  lane l holds row l%32, k = 8*(l/32) + j
//              B[16x32]  lane l holds col l%32, k = 8*(l/32) + j
//              D[32x32]  lane l holds col l%32, rows 8*(r/4) + 4*(l/32) + r%4 (r = 0..15)
// A sum over k does not depend on the order of k, so a kernel may feed any fixed permutation of the k index as long
// as the A and B operands of one instruction use the same one. The kernels use this to feed accumulator tiles
// (D layout) straight back in as B operands without a trip through LDS.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
// Native 32-bit integer vectors for raw 16 / 8-byte moves: unlike HIP's uint4 / uint2 structs they always stay in
// registers (a select or copy of the struct types can leave an array of them in scratch memory).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Kernel entry: fetch the listed kernel arguments into scalar registers in one batch. Scalar loads complete out of
// order, so every wait for one of them waits for all of them. An argument the compiler would fetch later (behind a
// branch, or after a value read from device memory) costs one more memory round trip before the kernel's first
// load; an empty asm that takes them all as scalar operands makes the compiler fetch them together.
#define Q35_SGPR_OPERAND(a) "s"(a)
#define Q35_FE_1(m, a) m(a)
#define Q35_FE_2(m, a, ...) m(a), Q35_FE_1(m, __VA_ARGS__)
#define Q35_FE_3(m, a, ...) m(a), Q35_FE_2(m, __VA_ARGS__)
#define Q35_FE_4(m, a, ...) m(a), Q35_FE_3(m, __VA_ARGS__)
#define Q35_FE_5(m, a, ...) m(a), Q35_FE_4(m, __VA_ARGS__)
#define Q35_FE_6(m, a, ...) m(a), Q35_FE_5(m, __VA_ARGS__)
#define Q35_FE_7(m, a, ...) m(a), Q35_FE_6(m, __VA_ARGS__)
#define Q35_FE_8(m, a, ...) m(a), Q35_FE_7(m, __VA_ARGS__)
#define Q35_FE_9(m, a, ...) m(a), Q35_FE_8(m, __VA_ARGS__)
#define Q35_FE_10(m, a, ...) m(a), Q35_FE_9(m, __VA_ARGS__)
#define Q35_FE_11(m, a, ...) m(a), Q35_FE_10(m, __VA_ARGS__)
#define Q35_FE_12(m, a, ...) m(a), Q35_FE_11(m, __VA_ARGS__)
#define Q35_FE_13(m, a, ...) m(a), Q35_FE_12(m, __VA_ARGS__)
#define Q35_FE_14(m, a, ...) m(a), Q35_FE_13(m, __VA_ARGS__)
#define Q35_FE_15(m, a, ...) m(a), Q35_FE_14(m, __VA_ARGS__)
#define Q35_FE_16(m, a, ...) m(a), Q35_FE_15(m, __VA_ARGS__)
#define Q35_FE_17(m, a, ...) m(a), Q35_FE_16(m, __VA_ARGS__)
#define Q35_FE_18(m, a, ...) m(a), Q35_FE_17(m, __VA_ARGS__)
#define Q35_FE_19(m, a, ...) m(a), Q35_FE_18(m, __VA_ARGS__)
#define Q35_FE_20(m, a, ...) m(a), Q35_FE_19(m, __VA_ARGS__)
#define Q35_FE_21(m, a, ...) m(a), Q35_FE_20(m, __VA_ARGS__)
#define Q35_FE_22(m, a, ...) m(a), Q35_FE_21(m, __VA_ARGS__)
#define Q35_FE_23(m, a, ...) m(a), Q35_FE_22(m, __VA_ARGS__)
#define Q35_FE_24(m, a, ...) m(a), Q35_FE_23(m, __VA_ARGS__)
#define Q35_FE_PICK(_1, _2, _3, _4, _5, _6, _7, _8, _9, _10, _11, _12, _13, _14, _15, _16, _17, _18, _19, _20, _21, _22, _23, _24, NAME, ...) NAME
#define Q35_FOR_EACH(m, ...) Q35_FE_PICK(__VA_ARGS__, Q35_FE_24, Q35_FE_23, Q35_FE_22, Q35_FE_21, Q35_FE_20, Q35_FE_19, Q35_FE_18, Q35_FE_17, Q35_FE_16, Q35_FE_15, Q35_FE_14, Q35_FE_13, Q35_FE_12, Q35_FE_11, Q35_FE_10, Q35_FE_9, Q35_FE_8, Q35_FE_7, Q35_FE_6, Q35_FE_5, Q35_FE_4, Q35_FE_3, Q35_FE_2, Q35_FE_1)(m, __VA_ARGS__)
#define Q35_ARGS_UPFRONT(...) asm volatile("" ::Q35_FOR_EACH(Q35_SGPR_OPERAND, __VA_ARGS__))

namespace q35 {

// Element types the kernels accept for activations (q, k, v, o, gate).
enum DType : int { kF32 = 0, kBF16 = 1 };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__bf16 x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float x) { return (__bf16)x; }

// bf16 bit patterns -> fp32 (exact).
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { f32x4 z = {0.f, 0.f, 0.f, 0.f}; return z; }
__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Pack two 4-row accumulator fragments into one 8-element bf16 operand (k permutation described above).
__device__ __forceinline__ bf16x8 pack8(const f32x4& lo, const f32x4& hi) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) { r[i] = (__bf16)lo[i]; r[4 + i] = (__bf16)hi[i]; }
  return r;
}

// sigmoid with the hardware reciprocal (v_rcp_f32, 1 ulp) in place of an IEEE division (the attention output gate,
// one per output value, and the GDN beta). Every kernel uses this one form, so fused forms round as their parts.
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
// x = hi + lo up to 2^-17 |x|: hi = bf16(x), lo = bf16(x - hi), both rounded to nearest even (the split of fp32
// activations for the int8 GEMM's bf16 products). The subtraction is never contracted into the product that made x
// (an FMA would form lo from the unrounded product): every producer of split values rounds the same way.
struct bf16_hl {
  __bf16 hi, lo;
};
__device__ __forceinline__ bf16_hl bf16_split(float x) {
#pragma clang fp contract(off)
  const __bf16 h = (__bf16)x;
  return {h, (__bf16)(x - (float)h)};
}
// silu(x) = x / (1 + e^-x) with the hardware reciprocal (v_rcp_f32, 1 ulp) in place of an IEEE division (about ten
// VALU instructions); large negative x gives -0 and x = -inf NaN, as the division does. Every kernel uses this one
// form, so kernels that are compared bit for bit (a fused form against its parts) round alike.
__device__ __forceinline__ float silu_f(float x) { return x * __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : log1pf(__expf(x)); }  // threshold 20

// Block barrier that orders LDS traffic only. __syncthreads() also waits for every outstanding global load of the
// calling wave (its fence has release semantics), which would drain register prefetches issued for the next
// iteration; this waits for LDS operations (lgkmcnt) and meets the other waves, leaving global loads in flight.
// The "memory" clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Sum / max over the 64 lanes of a wave (butterfly; every lane ends with the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace q35
