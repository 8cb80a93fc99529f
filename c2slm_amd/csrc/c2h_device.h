// Device-side scalar helpers shared by the gfx950 kernels.
//
// Every helper reproduces one scalar operation of the reference's CPU path
// bit for bit.  The whole library is compiled with -ffp-contract=off, so
// a*b+c is always two roundings unless written as __builtin_fmaf (used only
// where the reference calls archsimd MulAdd).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace c2h {

// f(std::integral_constant<int, i>) for i = 0..N-1, expanded in the source:
// arrays indexed by i are promoted to registers even when they stay live
// across a loop (an unrolled `for` can leave such an array in scratch memory).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

constexpr int QK_K = 256;
constexpr int BS_Q4K = 144;
constexpr int BS_Q6K = 210;
constexpr int BS_Q6K_PACKED = 208;  // ql|qh|scales; d lives in a separate fp16 array
constexpr int BS_Q8K = 292;
constexpr int QK8_0 = 32;
constexpr int BS_Q8_0 = 34;
constexpr int BS_Q5_0 = 22;
constexpr int MAX_Q8K_BLOCKS = 64;  // 16384 columns, the reference pool's Q8_K scratch (engine/pool.go:59)

enum GgmlType : int { T_F32 = 0, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };

__device__ __forceinline__ float bits_f32(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f32_bits(float f) { return __float_as_uint(f); }

// fp16 -> f32 with the semantics of the simd kernels' lookup table
// (internal/simd/c2_tensor_dot_q8_0_gen.go:24-66): both zeros give +0,
// subnormals are exact, Inf/NaN keep their payload.
__device__ __forceinline__ float fp16_simd(uint32_t h) {
  uint32_t sign = (h >> 15) << 31;
  uint32_t e = (h >> 10) & 31u;
  uint32_t m = h & 0x3ffu;
  if (e == 0) {
    if (m == 0) return 0.0f;
    float f = (float)m * 0x1p-24f;  // exact: m < 2^10
    return sign ? -f : f;
  }
  if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

// c ? a : b as mask arithmetic: the compiler turns some ternaries on
// per-lane conditions into divergent branches, which this cannot become.
__device__ __forceinline__ uint32_t blend_u32(bool c, uint32_t a, uint32_t b) {
  const uint32_t m = 0u - (uint32_t)c;
  return (a & m) | (b & ~m);
}

// fp16_simd without branches (identical bits): blends the subnormal, normal
// and Inf/NaN encodings, so a per-lane value never splits the wave.
__device__ __forceinline__ float fp16_simd_nb(uint32_t h) {
  const uint32_t sign = (h >> 15) << 31;
  const uint32_t e = (h >> 10) & 31u;
  const uint32_t m = h & 0x3ffu;
  // subnormal (or zero): m * 2^-24 is exact; both zeros give +0
  const uint32_t sub = __float_as_uint((float)m * 0x1p-24f) | blend_u32(m != 0u, sign, 0u);
  const uint32_t normal = sign | ((e + 112u) << 23) | (m << 13);
  const uint32_t special = sign | 0x7f800000u | (m << 13);
  return bits_f32(blend_u32(e == 0u, sub, blend_u32(e == 31u, special, normal)));
}

// tensor.FP16ToF32 (tensor/fp16.go:16-50): as above but -0 keeps its sign.
__device__ __forceinline__ float fp16_tensor(uint32_t h) {
  if ((h & 0x7fffu) == 0) return bits_f32((h >> 15) << 31);
  return fp16_simd(h);
}

// archsimd ConvertToInt32 (VCVTTPS2DQ): truncation, INT32_MIN for NaN or
// out-of-range lanes.
__device__ __forceinline__ int32_t x86_cvtt_i32(float t) {
  if (!(t >= -2147483648.0f && t < 2147483648.0f)) return INT32_MIN;
  return (int32_t)t;
}

// One lane of internal/simd/c2_tensor_swiglu_gen.go:11-51.
__device__ __forceinline__ float swiglu_poly(float xv, float up) {
  const float half = bits_f32(0x3f000000u), one = bits_f32(0x3f800000u);
  const float inv_ln2 = bits_f32(0x3fb8aa3bu), ln2 = bits_f32(0x3f317218u);
  const float c5 = bits_f32(0x3c088888u), c4 = bits_f32(0x3d2aaaabu), c3 = bits_f32(0x3e2aaaabu);
  float nx = -xv;
  float nf = nx * inv_ln2;
  int32_t np = x86_cvtt_i32(nf + half);
  int32_t nn = x86_cvtt_i32(nf - half);
  int32_t ni = (nf >= 0.0f) ? np : nn;
  ni = ni < -126 ? -126 : ni;
  ni = ni > 127 ? 127 : ni;
  float nif = (float)ni;
  float r = nx - (nif * ln2);
  float p = c5 * r;
  p = p + c4;
  p = p * r;
  p = p + c3;
  p = p * r;
  p = p + half;
  p = p * r;
  p = p + one;
  p = p * r;
  p = p + one;
  float sc = bits_f32((uint32_t)(ni + 127) << 23);
  float ev = p * sc;
  float den = one + ev;
  float sig = one / den;
  float silu = xv * sig;
  return silu * up;
}

// The scalar tail of the same file (:53-57), for the last n%8 elements.
__device__ __forceinline__ float swiglu_tail(float g32, float up) {
  double g = (double)g32;
  float silu = (float)(g / (1.0 + exp(-g)));
  return silu * up;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// ---- wave64 reductions through DPP (VALU lane moves, no LDS round trip)

enum : int {
  DPP_QUAD_1032 = 0xB1,   // quad_perm [1,0,3,2]
  DPP_QUAD_2301 = 0x4E,   // quad_perm [2,3,0,1]
  DPP_HALF_MIRROR = 0x141,
  DPP_MIRROR = 0x140,
  DPP_BCAST15 = 0x142,
  DPP_BCAST31 = 0x143,
};

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xf, false);
}
// The same move with 0 in lanes the control leaves out: 0 is the identity of
// the max of non-negative values and of sums, which lets the compiler fold
// the move into the following VALU op (one v_*_dpp instruction, no copy).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp0_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL, ROW_MASK>(__float_as_int(v)));
}

__device__ __forceinline__ float fmax_gt(float a, float b) { return (b > a) ? b : a; }

// Max over the 64 lanes of values that are never NaN ('>' semantics, so a
// -0 never replaces +0); the result is returned in every lane.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmax_gt(v, dpp_f<DPP_QUAD_1032>(v));
  v = fmax_gt(v, dpp_f<DPP_QUAD_2301>(v));
  v = fmax_gt(v, dpp_f<DPP_HALF_MIRROR>(v));
  v = fmax_gt(v, dpp_f<DPP_MIRROR>(v));
  v = fmax_gt(v, dpp_f<DPP_BCAST15, 0xa>(v));
  v = fmax_gt(v, dpp_f<DPP_BCAST31, 0xc>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte non-temporal load: for the vocab matrix, which is read once per
// step and would otherwise push the layer weights out of the last-level
// cache (the layer kernels use plain loads so that cache keeps them).
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
  u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
typedef float f32x4_t __attribute__((ext_vector_type(4)));


}  // namespace c2h
