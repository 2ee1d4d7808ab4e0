// Self-test kernels: the hardware-rounded primitives of remnant_device.h
// (the functions the pack, reconstruct and decode kernels call) evaluated over
// their whole input domains, for the GPU tests to compare with the software
// rounding and with the CPU oracle. Test infrastructure, built into its own
// library (libremnant_selftest.so); the product library does not contain it.
#include "remnant_device.h"

using namespace rm;

namespace {

constexpr int kBlocks = 4096;
constexpr int kThreads = 256;

// Add a per-thread mismatch count to result[0] (one atomic per wave) and
// lower result[1] to the smallest mismatching input.
__device__ void report(unsigned long long* result, unsigned long long bad, uint64_t first_bad) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) bad += __shfl_xor(bad, d, 64);
  if ((threadIdx.x & 63) == 0 && bad) atomicAdd(result, bad);
  if (first_bad != ~0ull) atomicMin(result + 1, first_bad);
}

// FP32 -> BF16 pair conversion vs bf16_rne over inputs [first, first + count).
__global__ __launch_bounds__(kThreads) void bf16_pair_kernel(uint64_t first, uint64_t count,
                                                             unsigned long long* result) {
  unsigned long long bad = 0;
  uint64_t first_bad = ~0ull;
  for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; 2 * i < count;
       i += (uint64_t)gridDim.x * kThreads) {
    const uint64_t u0 = first + 2 * i, u1 = u0 + 1 < first + count ? u0 + 1 : u0;
    const float a = u2f((uint32_t)u0), b = u2f((uint32_t)u1);
    const uint32_t hw = __builtin_bit_cast(uint32_t, bf16_pair(a, b));
    const bool nan_a = ((uint32_t)u0 & 0x7fffffffu) > 0x7f800000u;
    const bool nan_b = ((uint32_t)u1 & 0x7fffffffu) > 0x7f800000u;
    if (!nan_a && (hw & 0xffffu) != bf16_rne(a)) {
      ++bad;
      first_bad = first_bad < u0 ? first_bad : u0;
    }
    if (!nan_b && u1 != u0 && (hw >> 16) != bf16_rne(b)) {
      ++bad;
      first_bad = first_bad < u1 ? first_bad : u1;
    }
  }
  report(result, bad, first_bad);
}

// Scaled FP8 encode: out[(e - e_lo) * 65536 + n] = code of BF16 pattern n at
// scale 2^e (byte 0 of the pair conversion; both halves are checked equal).
__global__ __launch_bounds__(kThreads) void fp8_encode_kernel(int e_lo, int e_count,
                                                              uint8_t* out,
                                                              unsigned long long* result) {
  unsigned long long bad = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < (uint64_t)e_count * 65536;
       i += (uint64_t)gridDim.x * kThreads) {
    const int e = e_lo + (int)(i >> 16);
    const uint16_t n = (uint16_t)(i & 0xffffu);
    const __bf16 v = __builtin_bit_cast(__bf16, n);
    s16x2 acc = {0, 0};
    acc = fp8_pair<false>(acc, bf16x2{v, v}, exp2i(e));
    acc = fp8_pair<true>(acc, bf16x2{v, v}, exp2i(e));
    const uint32_t w = __builtin_bit_cast(uint32_t, acc);
    if ((w & 0xff) != ((w >> 8) & 0xff) || (w & 0xffff) != (w >> 16)) ++bad;
    out[i] = (uint8_t)(w & 0xffu);
  }
  report(result, bad, ~0ull);
}

// Scaled FP8 decode: out[s * 256 + c] = BF16 bits of code c at scale byte s
// (2^(s - 127)), s in 1..254 (0 for s = 0 and 255).
__global__ __launch_bounds__(kThreads) void fp8_decode_kernel(uint16_t* out) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= 256 * 256) return;
  const int s = i >> 8, c = i & 255;
  uint16_t r = 0;
  if (s >= 1 && s <= 254) {
    const uint32_t codes = (uint32_t)c | ((uint32_t)c << 8);
    r = (uint16_t)(fp8_pair_to_bf16<false>(codes, exp2i(s - 127)) & 0xffffu);
  }
  out[i] = r;
}

// Neighbouring floats of a positive finite v.
__device__ __forceinline__ double below(float v) { return (double)u2f(f2u(v) - 1); }
__device__ __forceinline__ double above(float v) { return (double)u2f(f2u(v) + 1); }

// Correct rounding of the store's root and reciprocal, proved exactly for FP32
// bit patterns [first, end) (positive finite x): s = RN(sqrt(x)) iff x lies
// strictly between the squares of the midpoints around s, and r = RN(1 / s)
// iff 1 lies strictly between s times the midpoints around r. Midpoints of
// adjacent floats have 25 significant bits, so the midpoints and these
// products are exact in double precision, and no tie can occur.
__global__ __launch_bounds__(kThreads) void inv_root_kernel(uint32_t first, uint32_t end,
                                                            unsigned long long* result) {
  unsigned long long bad = 0;
  uint64_t first_bad = ~0ull;
  for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; first + i < end;
       i += (uint64_t)gridDim.x * kThreads) {
    const uint32_t xb = first + (uint32_t)i;
    const float x = u2f(xb);
    const float s = root_rn(x);
    const float r = inv_root(x);
    const double ds = s, dr = r, dx = x;
    const double slo = 0.5 * (ds + below(s)), shi = 0.5 * (ds + above(s));
    const double rlo = 0.5 * (dr + below(r)), rhi = 0.5 * (dr + above(r));
    const bool ok = slo * slo < dx && dx < shi * shi && rlo * ds < 1.0 && 1.0 < rhi * ds;
    if (!ok) {
      ++bad;
      first_bad = first_bad < xb ? first_bad : xb;
    }
  }
  report(result, bad, first_bad);
}

// Per-element RMS reciprocal of the store: r = RN(1 / RN(sqrt(sumsq / 512 + eps))).
__global__ __launch_bounds__(kThreads) void inv_rms_kernel(const float* sumsq, const float* eps,
                                                           float* out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    out[i] = inv_root(sumsq[i] * (1.0f / 512.0f) + eps[i]);
}

// The BF16 pair conversion of an array: out[i] = BF16 bits of x[i] (n even).
__global__ __launch_bounds__(kThreads) void bf16_array_kernel(const float* x, uint32_t* out,
                                                              int64_t pairs) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < pairs;
       i += (int64_t)gridDim.x * kThreads)
    out[i] = __builtin_bit_cast(uint32_t, bf16_pair(x[2 * i], x[2 * i + 1]));
}

// RoPE rotation of the Direct decode's position mode: out[2 (p * 32 + j)] and
// out[2 (p * 32 + j) + 1] = cos and sin of RN(pos * theta[j]), pos = p * step.
__global__ __launch_bounds__(kThreads) void rope_cs_kernel(const float* theta, int64_t n_pos,
                                                           int step, float* out) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_pos * kRopePairs;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t p = i / kRopePairs;
    const float x = (float)(p * step) * theta[i - p * kRopePairs];
    float s, c;
    rope_sincos(x, s, c);
    out[2 * i] = c;
    out[2 * i + 1] = s;
  }
}

// Largest |v_sin_f32(f) - sin(2 pi f)| and |v_cos_f32(f) - cos(2 pi f)| (in
// double) over the FP32 bit patterns [first, end) of one sign: err[0] and
// err[1] as float bit patterns (non-negative floats order as integers).
__global__ __launch_bounds__(kThreads) void sincos_error_kernel(uint32_t first, uint32_t end,
                                                                unsigned int* err) {
  float es = 0.0f, ec = 0.0f;
  for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; first + i < end;
       i += (uint64_t)gridDim.x * kThreads) {
    const float f = u2f(first + (uint32_t)i);
    const double a = (double)f * 6.283185307179586476925286766559;
    es = fmaxf(es, (float)fabs((double)__builtin_amdgcn_sinf(f) - sin(a)));
    ec = fmaxf(ec, (float)fabs((double)__builtin_amdgcn_cosf(f) - cos(a)));
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    es = fmaxf(es, __shfl_xor(es, d, 64));
    ec = fmaxf(ec, __shfl_xor(ec, d, 64));
  }
  if ((threadIdx.x & 63) == 0) {
    atomicMax(err, f2u(es));
    atomicMax(err + 1, f2u(ec));
  }
}

// Gather ceiling of a sparse decode's record reads (a bench calibration, not
// part of the product library): every valid top-k entry of every token is
// resolved through the block table like the decode resolves it (entry r of
// token t: request t / q_len, page block_table[b, r / 64], row r % 64), then
// the record bytes the decode copies are read with all of a wave's loads in
// flight -- Packed: the 21 aligned 16-byte pieces covering the 328-byte record
// (from 8 bytes before an odd row); Native: the 36 pieces of the 576-byte data
// row and the 16-byte piece holding its scale row -- and folded by XOR into
// one word per wave. Nothing else is done, so its time bounds what the
// decode's memory side can reach on the same entries. Invalid entries (k >=
// length, r < 0, r >= seqlen, no page) read nothing.
template <bool kPacked>
__global__ __launch_bounds__(256) void gather_ceiling_kernel(
    const uint8_t* __restrict__ pool, int64_t pool_pages, const int32_t* __restrict__ block_table,
    int64_t bt_stride, int64_t max_blocks, const int32_t* __restrict__ seqlens,
    const int32_t* __restrict__ indices, int64_t topk, const int32_t* __restrict__ topk_length,
    int64_t q_len, int64_t tokens, uint32_t* __restrict__ out) {
  constexpr int kPieces = kPacked ? 21 : 37;
  constexpr int kPage = kPacked ? kPageBytes : kNativePageBytes;
  const int lane = wave_lane();
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t waves = (int64_t)gridDim.x * 4;
  const int64_t groups_per_token = (topk + 63) / 64;
  uint32_t acc = 0;
  for (int64_t gi = wave; gi < tokens * groups_per_token; gi += waves) {
    const int64_t t = gi / groups_per_token, k = (gi - t * groups_per_token) * 64 + lane;
    const int64_t b = t / q_len;
    int64_t len = topk_length ? topk_length[t] : topk;
    len = len < topk ? len : topk;
    uint64_t base = 0;  // 0: nothing to read
    if (k < len) {
      const int64_t r = indices[t * topk + k];
      const int64_t seq = seqlens ? seqlens[b] : INT64_MAX;
      if (r >= 0 && r < seq && (r >> 6) < max_blocks) {
        const int64_t page = block_table[b * bt_stride + (r >> 6)];
        if (page >= 0 && page < pool_pages) {
          const int row = (int)(r & 63);
          const uint8_t* pg = pool + page * kPage;
          base = kPacked ? (uint64_t)(pg + row * kRecordBytes) & ~(uint64_t)15
                         : (uint64_t)(pg + row * kNativeDataBytes);
          if (!kPacked) base |= (uint64_t)row << 58;  // the scale row's index, top bits
        }
      }
    }
    // 64 records x kPieces pieces: load j covers pieces 64 j .. 64 j + 63 of the
    // group, lane -> (record, piece) = divmod(64 j + lane, kPieces)
    u32x4 v[kPieces];
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      const int c = 64 * j + lane;
      const int rec = c / kPieces, piece = c - rec * kPieces;
      const uint64_t rb = __shfl(base, rec, 64);
      v[j] = u32x4{0u, 0u, 0u, 0u};
      if (rb) {
        const uint64_t addr = rb & (((uint64_t)1 << 58) - 1);
        const uint8_t* src;
        if (kPacked || piece < 36) {
          src = (const uint8_t*)addr + 16 * piece;
        } else {  // Native scale row: page + 64 data rows + row * 8, in its 16-byte piece
          const int row = (int)(rb >> 58);
          src = (const uint8_t*)(addr - (uint64_t)row * kNativeDataBytes +
                                 kPageRecords * kNativeDataBytes + ((row * kScaleBytes) & ~15));
        }
        v[j] = __builtin_nontemporal_load((const u32x4*)src);
      }
    }
#pragma unroll
    for (int j = 0; j < kPieces; ++j) acc ^= v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3];
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) acc ^= __shfl_xor(acc, d, 64);
  if (lane == 0) out[wave] = acc;
}

int status() { return hipGetLastError() == hipSuccess ? 0 : -6; }

}  // namespace

// result: device [2] u64, initialised to {0, ~0} by the caller.
extern "C" int rmt_bf16_pair_mismatches(uint64_t first, uint64_t count,
                                        unsigned long long* result, void* stream) {
  if (first + count > (1ull << 32)) return -2;
  hipLaunchKernelGGL(bf16_pair_kernel, dim3(kBlocks), dim3(kThreads), 0, (hipStream_t)stream,
                     first, count, result);
  return status();
}

// out: device [(e_hi - e_lo + 1) * 65536] u8; result as above (pair halves that differ).
extern "C" int rmt_fp8_encode_table(int e_lo, int e_hi, uint8_t* out, unsigned long long* result,
                                    void* stream) {
  if (e_lo < -126 || e_hi > 127 || e_hi < e_lo) return -2;
  hipLaunchKernelGGL(fp8_encode_kernel, dim3(kBlocks), dim3(kThreads), 0, (hipStream_t)stream,
                     e_lo, e_hi - e_lo + 1, out, result);
  return status();
}

// out: device [256 * 256] u16.
extern "C" int rmt_fp8_decode_table(uint16_t* out, void* stream) {
  hipLaunchKernelGGL(fp8_decode_kernel, dim3(256), dim3(kThreads), 0, (hipStream_t)stream, out);
  return status();
}

extern "C" int rmt_inv_root_mismatches(uint32_t first, uint32_t end, unsigned long long* result,
                                       void* stream) {
  if (end < first) return -2;
  hipLaunchKernelGGL(inv_root_kernel, dim3(kBlocks), dim3(kThreads), 0, (hipStream_t)stream,
                     first, end, result);
  return status();
}

extern "C" int rmt_inv_rms(const float* sumsq, const float* eps, float* out, int64_t n,
                           void* stream) {
  if (n < 0) return -2;
  if (n == 0) return 0;
  hipLaunchKernelGGL(inv_rms_kernel, dim3(kBlocks), dim3(kThreads), 0, (hipStream_t)stream,
                     sumsq, eps, out, n);
  return status();
}

// out: device [n] u16 (n even).
extern "C" int rmt_bf16_array(const float* x, uint16_t* out, int64_t n, void* stream) {
  if (n < 0 || (n & 1)) return -2;
  if (n == 0) return 0;
  hipLaunchKernelGGL(bf16_array_kernel, dim3(kBlocks), dim3(kThreads), 0, (hipStream_t)stream, x,
                     (uint32_t*)out, n / 2);
  return status();
}

// out: device [n_pos * 32 * 2] f32; theta: device [32] f32.
extern "C" int rmt_rope_cos_sin(const float* theta, int64_t n_pos, int step, float* out,
                                void* stream) {
  if (n_pos < 0 || step < 0 || (double)n_pos * step >= 16777216.0) return -2;
  if (n_pos == 0) return 0;
  hipLaunchKernelGGL(rope_cs_kernel, dim3(kBlocks), dim3(kThreads), 0, (hipStream_t)stream, theta,
                     n_pos, step, out);
  return status();
}

// err: device [2] u32, zeroed by the caller.
extern "C" int rmt_sincos_error(uint32_t first, uint32_t end, unsigned int* err, void* stream) {
  if (end < first) return -2;
  hipLaunchKernelGGL(sincos_error_kernel, dim3(kBlocks), dim3(kThreads), 0, (hipStream_t)stream,
                     first, end, err);
  return status();
}

// The gather ceiling of a decode's record reads (see gather_ceiling_kernel);
// out: device [4 * blocks] u32, blocks = 1024 (one word per wave).
extern "C" int rmt_gather_ceiling(int packed, const uint8_t* pool, int64_t pool_pages,
                                  const int32_t* block_table, int64_t bt_stride,
                                  int64_t max_blocks, const int32_t* seqlens,
                                  const int32_t* indices, int64_t topk,
                                  const int32_t* topk_length, int64_t q_len, int64_t tokens,
                                  uint32_t* out, void* stream) {
  if (pool_pages < 0 || topk < 0 || q_len < 1 || tokens < 0 || bt_stride < max_blocks) return -2;
  if (tokens == 0 || topk == 0) return 0;
  const dim3 grid(1024), block(256);
  if (packed)
    hipLaunchKernelGGL(gather_ceiling_kernel<true>, grid, block, 0, (hipStream_t)stream, pool,
                       pool_pages, block_table, bt_stride, max_blocks, seqlens, indices, topk,
                       topk_length, q_len, tokens, out);
  else
    hipLaunchKernelGGL(gather_ceiling_kernel<false>, grid, block, 0, (hipStream_t)stream, pool,
                       pool_pages, block_table, bt_stride, max_blocks, seqlens, indices, topk,
                       topk_length, q_len, tokens, out);
  return status();
}
