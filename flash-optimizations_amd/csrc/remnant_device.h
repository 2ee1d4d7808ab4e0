// Device-side geometry and bit-exact scalar codec helpers shared by the
// pack, reconstruct and decode kernels (gfx950 / CDNA4, wave64).
//
// Record geometry (docs/agents/numerical-and-validation.md:10-12 in the
// reference): 512 coordinates = 448 NoPE + 64 RoPE tail; Packed keeps 256 as
// E4M3 codes + a 512-bit bitmap + 8 UE8M0 scales = 328 bytes, stored as one
// contiguous record (codes, bitmap, scales); a page holds 64 records, so a
// record starts 16-byte aligned (even rows) or 8 bytes past it (odd rows).
// Native records are 584 bytes: 448 E4M3 codes + 64 rotated BF16 + 8 scales; a
// Native page keeps its 64 data rows (576 bytes) followed by the 64 scale rows.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rm {

constexpr int kHeadDim = 512;
constexpr int kNopeDim = 448;
constexpr int kRopePairs = 32;
constexpr int kKeep = 256;
constexpr int kGroup = 64;
constexpr int kCodeBytes = 256;
constexpr int kBitmapBytes = 64;
constexpr int kDataBytes = kCodeBytes + kBitmapBytes;   // 320
constexpr int kScaleBytes = 8;
constexpr int kRecordBytes = kDataBytes + kScaleBytes;                        // 328
constexpr int kPageRecords = 64;
constexpr int kPageBytes = kPageRecords * kRecordBytes;                       // 20992
constexpr int kNativeDataBytes = kNopeDim + 2 * (kHeadDim - kNopeDim);       // 576
constexpr int kNativePageBytes = kPageRecords * (kNativeDataBytes + kScaleBytes);  // 37376

// Where the Packed records of a pool live. Contiguous pages: `values` is the
// pool; a page holds 64 records back to back, so slot s starts s * (K + 72)
// bytes in (the other two pointers are unused). Planes (the reference's pool
// tensors values u8 [rows, K], bitmaps u64 [rows, 8], scales u8 [rows, 8],
// candidate-sglang.patch:900-904): the three parts of slot s are row s of
// each plane.
struct PackedSrc {
  const uint8_t* values;
  const uint8_t* bitmaps;
  const uint8_t* scales;
};
struct PackedDst {  // the same, written by the store
  uint8_t* values;
  uint8_t* bitmaps;
  uint8_t* scales;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// float -> bf16 bits, round to nearest even (inputs are finite here).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  uint32_t u = f2u(f);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return u2f(h << 16); }

// OCP E4M3 (e4m3fn) encode, round to nearest even, |q| <= 448 by construction.
__device__ __forceinline__ uint32_t e4m3_rne(float q) {
  uint32_t b = f2u(q);
  uint32_t sign = (b >> 24) & 0x80u;
  uint32_t ab = b & 0x7fffffffu;
  uint32_t code;
  if (u2f(ab) < 0x1p-6f) {
    code = (uint32_t)(int)__builtin_rintf(u2f(ab) * 512.0f);  // subnormal: m * 2^-9
  } else {
    uint32_t r = ab + 0x7ffffu + ((ab >> 20) & 1u);
    code = (r >> 20) - ((127u - 7u) << 3);
  }
  return sign | code;
}

// E4M3 code -> float (exact).
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  uint32_t e = (c >> 3) & 15u, m = c & 7u;
  float v = e ? u2f(((e + 120u) << 23) | (m << 20)) : (float)m * 0x1p-9f;
  return (c & 0x80u) ? -v : v;
}

// UE8M0 exponent: smallest e with max(amax, 1e-4) <= 448 * 2^e, i.e.
// ceil(log2(max(amax, 1e-4) / 448)).
__device__ __forceinline__ int ue8m0_exponent(float amax) {
  if (!(amax >= 1e-4f)) return -22;
  uint32_t b = f2u(amax);
  return (int)((b >> 23) & 0xffu) - 127 - 8 + ((b & 0x7fffffu) > 0x600000u ? 1 : 0);
}

// 2^e as a float for e in [-126, 127].
__device__ __forceinline__ float exp2i(int e) { return u2f((uint32_t)(e + 127) << 23); }

__device__ __forceinline__ int wave_lane() { return (int)(threadIdx.x & 63u); }

// Make a per-wave value provably uniform (scalar register).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Order LDS writes of a wave before later reads by other lanes of the same wave.
// The fences cover LDS only, so outstanding global loads are not waited for.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// ---- hardware-rounded primitives ----------------------------------------
// Each equals the software rounding above on its whole input domain; the
// self-test library (selftest.hip) checks that exhaustively on the GPU.

// Two floats -> packed BF16, round to nearest even (v_cvt_pk_bf16_f32; equal
// to bf16_rne for every non-NaN input).
__device__ __forceinline__ bf16x2 bf16_pair(float a, float b) {
  return bf16x2{(__bf16)a, (__bf16)b};
}

// E4M3 codes of a BF16 pair divided by a power-of-two scale, RNE, into byte
// pair 0 (kHi false) or 1 of `acc` (v_cvt_scalef32_pk_fp8_bf16; equal to
// e4m3_rne(n / scale) for every finite BF16 n with |n / scale| <= 448).
template <bool kHi>
__device__ __forceinline__ s16x2 fp8_pair(s16x2 acc, bf16x2 n, float scale) {
  return __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(acc, n, scale, kHi);
}

// Two E4M3 codes (bytes 0-1, or 2-3 with kHi) times a power-of-two scale ->
// two BF16 (v_cvt_scalef32_pk_bf16_fp8; equal to rounding the exact product
// code * scale to BF16 for every finite code and every UE8M0 scale the store
// writes).
template <bool kHi>
__device__ __forceinline__ uint32_t fp8_pair_to_bf16(uint32_t codes, float scale) {
  bf16x2 r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(codes, scale, kHi);
  return __builtin_bit_cast(uint32_t, r);
}

// RN(1 / RN(sqrt(x))) for x = sumsq / 512 + eps (wave-uniform). v_sqrt_f32
// alone is not the correctly rounded root (for x = 1e-6 it returns the lower
// neighbour of RN(sqrt(x))) but lies within one ulp of it. For 2^-96 <= x <
// 2^128 the root s = v_sqrt_f32(x) is corrected by the exact FMA residuals
// x - s' s of its neighbours s' (lower neighbour if x - s_dn s <= 0, upper if
// x - s_up s > 0): the steps the compiler's correctly rounded square root
// takes in that range, where it needs neither its scaling of tiny inputs nor
// its zero and infinity cases. There the root lies in [2^-48, 2^64), where one
// Newton step from v_rcp_f32, fma(fma(-s, r0, 1), r0, r0), equals the
// correctly rounded 1 / s. Other x take the compiler's square root and the
// correctly rounded division.
__device__ __forceinline__ bool inv_root_fast_range(uint32_t xb) {
  return xb - 0x0f800000u < 0x7f800000u - 0x0f800000u;
}
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }
__device__ __forceinline__ float sqrt_rn_normal(float x) {
  const float s = __builtin_amdgcn_sqrtf(x);
  const float sdn = u2f(f2u(s) - 1u);
  const float sup = u2f(f2u(s) + 1u);
  const float rdn = __builtin_fmaf(-sdn, s, x);
  const float rup = __builtin_fmaf(-sup, s, x);
  const float t = rdn <= 0.0f ? sdn : s;
  return rup > 0.0f ? sup : t;
}
// the correctly rounded root as the store computes it
__device__ __forceinline__ float root_rn(float x) {
  return inv_root_fast_range(__float_as_uint(x)) ? sqrt_rn_normal(x) : sqrt_rn(x);
}
__device__ __forceinline__ float recip_newton(float s) {
  const float r0 = __builtin_amdgcn_rcpf(s);
  return __builtin_fmaf(__builtin_fmaf(-s, r0, 1.0f), r0, r0);
}
__device__ __forceinline__ float inv_root(float x) {
  return inv_root_fast_range(__float_as_uint(x)) ? recip_newton(sqrt_rn_normal(x))
                                                 : 1.0f / sqrt_rn(x);
}
__device__ __forceinline__ float inv_rms(float sumsq, float eps) {
  const float x = sumsq * (1.0f / 512.0f) + eps;
  return inv_root(__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x))));
}

// cos and sin of a RoPE angle x = RN(pos * theta), for |x| < 2^24. The angle
// is first taken in revolutions, x / (2 pi), with 1 / (2 pi) split into a
// float kI1 = RN(1 / (2 pi)) and the remainder kI2 = RN(1 / (2 pi) - kI1): the
// product x * kI1 and its exact rounding error (one FMA) plus x * kI2 give the
// fractional revolutions f in [-1/2, 1/2] to about 2^-28 for |x| < 2^24 (the
// subtraction of the nearest integer is exact below 2^23 revolutions). The
// hardware v_sin_f32 / v_cos_f32, whose argument is in revolutions, then
// evaluate sin(2 pi f) and cos(2 pi f).
__device__ __forceinline__ void rope_sincos(float x, float& s, float& c) {
  constexpr float kI1 = 0x1.45f306p-3f;
  constexpr float kI2 = 0x1.b93910p-28f;
  const float ph = x * kI1;
  float pl = __builtin_fmaf(x, kI1, -ph);
  pl = __builtin_fmaf(x, kI2, pl);
  const float f = (ph - __builtin_rintf(ph)) + pl;
  s = __builtin_amdgcn_sinf(f);
  c = __builtin_amdgcn_cosf(f);
}

// Tail rotation of 4 interleaved (re, im) pairs held as floats, with
// (cos, sin) pairs from the frequency table: re' = xr*c - xi*s, im' = xr*s + xi*c,
// every product rounded (compiled without FMA contraction).
__device__ __forceinline__ void rope4(float* v, const float* cs) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float xr = v[2 * j], xi = v[2 * j + 1], c = cs[2 * j], s = cs[2 * j + 1];
    float a = xr * c, b = xi * s;
    float d = xr * s, e = xi * c;
    v[2 * j] = a - b;
    v[2 * j + 1] = d + e;
  }
}

}  // namespace rm
