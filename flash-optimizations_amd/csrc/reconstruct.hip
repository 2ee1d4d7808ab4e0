// Reconstruct: gather Packed records, dequantize to BF16 and rotate the tail.
//
// Semantics of unpack_gather_bf16 with the fused reader
// (candidate-sglang.patch:427-480 API, :502-588 gather/dequant, :590-668 fused
// RoPE): row (q, k) gathers slot physical[q, k]; invalid or padded selections
// give zero rows; dequantized values are BF16-rounded before the rotation;
// pruned partner lanes receive rotated values; frequency row = raw * 4.
//
// One wave64 per output row; lane l produces coordinates 8l..8l+7 and stores
// them as one 16-byte write, so a wave writes its 1 KiB row coalesced. The
// lane's codes are a contiguous run [rank, rank + popcount(byte)) of the code
// block, fetched with one 12-byte load and a funnel shift. The lanes owning the
// RoPE tail (56..63) hold whole (re, im) pairs, so the rotation needs no
// cross-lane traffic.
#include "remnant_device.h"
#include "remnant_mi355x.h"

using namespace rm;

namespace {

constexpr int kWaves = 4;

// Expand the kept codes of 8 coordinates (bitmap byte `bits`, MSB = first
// coordinate; codes = next bytes of `run`) to 8 floats scaled by 2^(s-127).
__device__ __forceinline__ void expand8(uint32_t bits, uint64_t run, float scale, float* v) {
  int used = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool kept = (bits >> (7 - i)) & 1u;
    const uint32_t code = (uint32_t)(run >> (8 * used)) & 0xffu;
    v[i] = kept ? e4m3_to_f32(code) * scale : 0.0f;
    used += kept ? 1 : 0;
  }
}

// Per-lane dequantization of a Packed record's coordinates 8l..8l+7 (pre-RoPE).
__device__ __forceinline__ void dequant_lane(const uint8_t* __restrict__ data,
                                             const uint8_t* __restrict__ scales, int lane,
                                             float* v) {
  // Bitmap words as little-endian 64-bit values; word w covers coords 64w..64w+63
  // (records are 8-byte aligned, so the words are read as 8-byte loads).
  const u32x2* bm = (const u32x2*)(data + kCodeBytes);
  uint32_t wlo[8], whi[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const u32x2 v = bm[w];
    wlo[w] = v[0];
    whi[w] = v[1];
  }
  const int word = lane >> 3, sub = lane & 7;
  int rank = 0;
  uint64_t mine = 0;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const uint64_t ww = ((uint64_t)whi[w] << 32) | wlo[w];
    rank += w < word ? __popcll(ww) : 0;
    mine = w == word ? ww : mine;
  }
  // coordinates before ours inside the word are its top 8*sub bits
  rank += sub ? __popcll(mine >> (64 - 8 * sub)) : 0;
  const uint32_t bits = (uint32_t)(mine >> (56 - 8 * sub)) & 0xffu;
  const int base = rank & ~3;
  const uint32_t* cw = (const uint32_t*)(data + base);
  const uint32_t d0 = cw[0], d1 = cw[1], d2 = cw[2];
  const uint32_t sh = 8u * (uint32_t)(rank & 3);
  const uint32_t lo = (uint32_t)((((uint64_t)d1 << 32) | d0) >> sh);
  const uint32_t hi = (uint32_t)((((uint64_t)d2 << 32) | d1) >> sh);
  const float scale = exp2i((int)scales[word] - 127);
  expand8(bits, ((uint64_t)hi << 32) | lo, scale, v);
}

__global__ __launch_bounds__(256) void unpack_gather_kernel(
    const uint8_t* __restrict__ pool, int64_t pool_rows, const int32_t* __restrict__ physical,
    int64_t ps_q, int64_t ps_k, const int32_t* __restrict__ raw, int64_t rs_q, int64_t rs_k,
    const int32_t* __restrict__ lengths, int64_t ls, int64_t nk, int64_t total,
    const float* __restrict__ freqs, int64_t freq_rows, uint16_t* __restrict__ out) {
  const int lane = wave_lane();
  const int wave = uniform((int)(threadIdx.x >> 6));
  for (int64_t row = (int64_t)blockIdx.x * kWaves + wave; row < total;
       row += (int64_t)gridDim.x * kWaves) {
    const int64_t q = row / nk, k = row - q * nk;
    const int64_t p = physical[q * ps_q + k * ps_k];
    bool valid = k < lengths[q * ls] && p >= 0 && p < pool_rows;
    int64_t r = 0;
    if (freqs) {
      r = raw[q * rs_q + k * rs_k];
      valid = valid && r >= 0 && r * 4 < freq_rows;
    }
    u32x4 o = {0u, 0u, 0u, 0u};
    if (valid) {
      const uint8_t* rec = pool + (p >> 6) * kPageBytes + (p & 63) * kRecordBytes;
      float v[8];
      dequant_lane(rec, rec + kDataBytes, lane, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = bf16_to_f32(bf16_rne(v[i]));
      if (freqs && lane >= kNopeDim / 8) {
        const float* f = freqs + (r * 4) * (2 * kRopePairs) + 8 * (lane - kNopeDim / 8);
        const f32x4 a = *(const f32x4*)f, b = *(const f32x4*)(f + 4);
        float cs[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        rope4(v, cs);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = bf16_rne(v[2 * i]) | (bf16_rne(v[2 * i + 1]) << 16);
    }
    *(u32x4*)(out + row * kHeadDim + 8 * lane) = o;
  }
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace

extern "C" int rm_unpack_gather_bf16(const uint8_t* pool, int64_t pool_pages,
                                     const int32_t* physical, int64_t physical_stride_q,
                                     int64_t physical_stride_k, const int32_t* raw,
                                     int64_t raw_stride_q, int64_t raw_stride_k,
                                     const int32_t* lengths, int64_t length_stride,
                                     int64_t n_queries, int64_t selected_k, const float* freqs,
                                     int64_t freq_rows, uint16_t* out, void* stream) {
  if (n_queries < 0 || selected_k < 0 || pool_pages < 0 || freq_rows < 0) return RM_ERR_SHAPE;
  const int64_t total = n_queries * selected_k;
  if (total == 0) return RM_OK;
  if (!pool || !physical || !lengths || !out || (freqs && !raw)) return RM_ERR_NULL;
  if (!aligned(pool, 16) || !aligned(out, 16) || (freqs && !aligned(freqs, 16)))
    return RM_ERR_ALIGN;
  int64_t blocks = (total + kWaves - 1) / kWaves;
  if (blocks > 256 * 64) blocks = 256 * 64;
  hipLaunchKernelGGL(unpack_gather_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, pool, pool_pages * kPageRecords, physical,
                     physical_stride_q, physical_stride_k, raw, raw_stride_q, raw_stride_k,
                     lengths, length_stride, selected_k, total, freqs, freq_rows, out);
  return hipGetLastError() == hipSuccess ? RM_OK : RM_ERR_LAUNCH;
}
