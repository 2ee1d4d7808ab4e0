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
// block, fetched with one 12-byte load and a byte funnel shift; v_perm places
// them (zeros for pruned coordinates) and v_cvt_scalef32_pk_bf16_fp8 applies
// the UE8M0 scale, producing BF16 directly. The lanes owning the RoPE tail
// (56..63) hold whole (re, im) pairs, so the rotation needs no cross-lane
// traffic.
//
// Survivor profiles other than 256 (64..448 in steps of 64) use the same
// scheme on (K + 72)-byte records: lanes 0..K/8-1 hold the codes, the next 8
// the bitmap words and the one after them the scales; the 448-survivor record
// (520 bytes) needs a 65th piece, which every lane loads from the same address.
#include "remnant_device.h"
#include "remnant_mi355x.h"

using namespace rm;

namespace {

constexpr int kWaves = 4;
constexpr int kRows = 4;  // rows per wave and loop iteration

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two E4M3 codes (bytes 0-1, or 2-3 with kHi) times scale -> two BF16. The
// hardware conversion equals BF16-rounding the FP32 product code * scale for
// every finite code and every finite UE8M0 scale.
template <bool kHi>
__device__ __forceinline__ uint32_t cvt2(uint32_t codes, float scale) {
  bf16x2 r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(codes, scale, kHi);
  return __builtin_bit_cast(uint32_t, r);
}

// Byte-addressed read of another lane's register (ds_bpermute).
__device__ __forceinline__ uint32_t from_lane(uint32_t v, int src_lane) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane << 2, (int)v);
}

// Exclusive prefix sum of x over the wave's lanes (row shifts within rows of 16,
// then row broadcasts 15 and 31).
__device__ __forceinline__ int wave_exclusive_sum(int x) {
  int v = x;
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false); // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false); // row_bcast:31
  return v - x;
}

// Per-lane dequantization of a kK-survivor record's coordinates 8l..8l+7
// (pre-RoPE) as 8 BF16 values. The record is held across the wave: lane i has
// bytes 8i..8i+7 (`piece`; for 256 survivors lanes 0-31 the codes, 32-39 the
// bitmap words, 40 the scales; `extra` holds bytes 512..519 when the record is
// longer than 512 bytes), so the lane's bitmap word, code run and scale are
// register reads from other lanes. `sel` maps a bitmap byte to the v_perm
// selectors that place its kept codes (the next bytes of the code run) and
// zeros for pruned slots.
template <int kK>
__device__ __forceinline__ u32x4 dequant_lane(u32x2 piece, u32x2 extra, int lane,
                                              const uint64_t* sel) {
  constexpr int kWordLane = kK / 8, kScaleLane = kK / 8 + 8;
  const int word = lane >> 3, sub = lane & 7;
  const uint32_t wlo = from_lane(piece[0], kWordLane + word);
  const uint32_t whi = from_lane(piece[1], kWordLane + word);
  const uint64_t mine = ((uint64_t)whi << 32) | wlo;  // coords 64 word .. 64 word + 63, MSB first
  // codes before the word: popcounts of the earlier words (carried by lane 8w+7)
  int rank = wave_exclusive_sum(sub == 7 ? __popcll(mine) : 0);
  // coordinates before ours inside the word are its top 8*sub bits
  rank += sub ? __popcll(mine >> (64 - 8 * sub)) : 0;
  const uint32_t bits = (uint32_t)(mine >> (56 - 8 * sub)) & 0xffu;
  // the lane's codes are the run [rank, rank + popcount(bits)): code dword k is
  // component k % 2 of lane k / 2
  const int a = rank >> 3;  // lane holding code bytes 8a..8a+7
  const uint32_t a0 = from_lane(piece[0], a), a1 = from_lane(piece[1], a);
  const uint32_t b0 = from_lane(piece[0], a + 1), b1 = from_lane(piece[1], a + 1);
  const bool odd = (rank >> 2) & 1;
  const uint32_t d0 = odd ? a1 : a0, d1 = odd ? b0 : a1, d2 = odd ? b1 : b0;
  const uint32_t lo4 = __builtin_amdgcn_alignbyte(d1, d0, (uint32_t)rank);  // low 2 bits used
  const uint32_t hi4 = __builtin_amdgcn_alignbyte(d2, d1, (uint32_t)rank);
  const uint64_t s = sel[bits];
  const uint32_t c03 = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)s);
  const uint32_t c47 = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)(s >> 32));
  // scale bytes: lane K/8 + 8 (a permute reads the value the source lane
  // offers, so both halves are read uniformly and selected here)
  const uint32_t sc_lo = kScaleLane < 64 ? __builtin_amdgcn_readlane(piece[0], kScaleLane & 63)
                                         : __builtin_amdgcn_readlane(extra[0], 0);
  const uint32_t sc_hi = kScaleLane < 64 ? __builtin_amdgcn_readlane(piece[1], kScaleLane & 63)
                                         : __builtin_amdgcn_readlane(extra[1], 0);
  const uint32_t sc = word < 4 ? sc_lo : sc_hi;
  const float scale = exp2i((int)((sc >> (8 * (word & 3))) & 0xffu) - 127);
  return u32x4{cvt2<false>(c03, scale), cvt2<true>(c03, scale), cvt2<false>(c47, scale),
               cvt2<true>(c47, scale)};
}

// Row indexing. The narrow form (every index and element offset below 2^31)
// keeps the per-row scalar work small: q = row / nk by a multiply-high with a
// host-computed magic number (round-up method; exact for all 32-bit rows).
struct Index {
  int64_t ps_q, ps_k, rs_q, rs_k, ls;  // element strides
  int64_t nk, total;
  uint32_t magic, shift;  // for nk >= 2
};

template <bool kNarrow>
__device__ __forceinline__ void split_row(int64_t row, const Index& ix, int64_t& q, int64_t& k) {
  if (kNarrow) {
    const uint32_t n = (uint32_t)row, d = (uint32_t)ix.nk;
    uint32_t qq = n;
    if (d > 1) {
      const uint32_t t = __umulhi(ix.magic, n);
      qq = (t + ((n - t) >> 1)) >> ix.shift;
    }
    q = qq;
    k = n - qq * d;
  } else {
    q = row / ix.nk;
    k = row - q * ix.nk;
  }
}

template <bool kNarrow, int kK>
__global__ __launch_bounds__(256) void unpack_gather_kernel(
    const uint8_t* __restrict__ pool, int64_t pool_rows, const int32_t* __restrict__ physical,
    const int32_t* __restrict__ raw, const int32_t* __restrict__ lengths, Index ix,
    const float* __restrict__ freqs, int64_t freq_rows, uint16_t* __restrict__ out) {
  static_assert(kK % 64 == 0 && kK >= 64 && kK <= 448, "survivor profiles are 64..448");
  constexpr int kBytes = kK + kBitmapBytes + kScaleBytes;  // K + 72
  constexpr int kPieces = kBytes / 8 < 64 ? kBytes / 8 : 64;
  // selector table: byte bits MSB-first = coordinates 0..7; selector byte i is
  // the rank of coordinate i among the kept ones, or 0x0c (a zero byte)
  __shared__ uint64_t sel[256];
  {
    const uint32_t e = threadIdx.x;
    uint32_t r = 0;
    uint64_t v = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool kept = (e >> (7 - i)) & 1u;
      v |= (uint64_t)(kept ? r : 0x0cu) << (8 * i);
      r += kept ? 1u : 0u;
    }
    sel[e] = v;
  }
  __syncthreads();
  const int lane = wave_lane();
  const int wave = uniform((int)(threadIdx.x >> 6));
  // kRows consecutive rows per wave and iteration: their index, bitmap and code
  // loads are issued together, so their latencies overlap
  for (int64_t row0 = ((int64_t)blockIdx.x * kWaves + wave) * kRows; row0 < ix.total;
       row0 += (int64_t)gridDim.x * kWaves * kRows) {
    const uint8_t* rec[kRows];
    int64_t rr[kRows];
    bool valid[kRows];
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      const int64_t row = row0 + j;
      int64_t q, k;
      split_row<kNarrow>(row < ix.total ? row : 0, ix, q, k);
      int64_t p, len, r = 0;
      if (kNarrow) {
        p = physical[(int32_t)q * (int32_t)ix.ps_q + (int32_t)k * (int32_t)ix.ps_k];
        len = lengths[(int32_t)q * (int32_t)ix.ls];
        if (freqs) r = raw[(int32_t)q * (int32_t)ix.rs_q + (int32_t)k * (int32_t)ix.rs_k];
      } else {
        p = physical[q * ix.ps_q + k * ix.ps_k];
        len = lengths[q * ix.ls];
        if (freqs) r = raw[q * ix.rs_q + k * ix.rs_k];
      }
      bool v = row < ix.total && k < len && p >= 0 && p < pool_rows;
      if (freqs) v = v && r >= 0 && r * 4 < freq_rows;
      const uint32_t pp = v ? (uint32_t)p : 0u;  // pool rows fit in int32
      rec[j] = pool + (uint64_t)(pp >> 6) * (kPageRecords * kBytes) + (pp & 63u) * kBytes;
      rr[j] = r;
      valid[j] = v;
    }
    // the whole record in one load: lane i reads bytes 8i..8i+7; the tail
    // lanes' frequency values are loaded in the same round trip
    u32x2 piece[kRows], extra[kRows];
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      piece[j] = u32x2{0u, 0u};
      extra[j] = u32x2{0u, 0u};
      if (valid[j] && lane < kPieces) piece[j] = *(const u32x2*)(rec[j] + 8 * lane);
      if (kBytes > 512 && valid[j]) extra[j] = *(const u32x2*)(rec[j] + 512);
    }
    f32x4 fa[kRows], fb[kRows];
    const bool tail = freqs && lane >= kNopeDim / 8;
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      fa[j] = f32x4{1.f, 0.f, 1.f, 0.f};
      fb[j] = f32x4{1.f, 0.f, 1.f, 0.f};
      if (tail && valid[j]) {
        const float* f = freqs + (rr[j] * 4) * (2 * kRopePairs) + 8 * (lane - kNopeDim / 8);
        fa[j] = *(const f32x4*)f;
        fb[j] = *(const f32x4*)(f + 4);
      }
    }
    u32x4 o[kRows];
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      o[j] = dequant_lane<kK>(piece[j], extra[j], lane, sel);
      if (!valid[j]) o[j] = u32x4{0u, 0u, 0u, 0u};
    }
    if (tail) {
#pragma unroll
      for (int j = 0; j < kRows; ++j) {
        if (!valid[j]) continue;
        // rotate the BF16 (re, im) pairs with the record's frequency row
        const f32x4 a = fa[j], b = fb[j];
        float cs[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[2 * i] = u2f(o[j][i] << 16);
          v[2 * i + 1] = u2f(o[j][i] & 0xffff0000u);
        }
        rope4(v, cs);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[j][i] = __builtin_bit_cast(uint32_t, bf16x2{(__bf16)v[2 * i], (__bf16)v[2 * i + 1]});
      }
    }
#pragma unroll
    for (int j = 0; j < kRows; ++j)
      if (row0 + j < ix.total) *(u32x4*)(out + (row0 + j) * kHeadDim + 8 * lane) = o[j];
  }
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

struct Launch {
  const uint8_t* pool;
  int64_t pool_rows;
  const int32_t *physical, *raw, *lengths;
  Index ix;
  const float* freqs;
  int64_t freq_rows;
  uint16_t* out;
};

template <int kK>
void launch_unpack(bool narrow, int64_t blocks, const Launch& a, hipStream_t s) {
  if (narrow)
    hipLaunchKernelGGL((unpack_gather_kernel<true, kK>), dim3((unsigned)blocks), dim3(256), 0, s,
                       a.pool, a.pool_rows, a.physical, a.raw, a.lengths, a.ix, a.freqs,
                       a.freq_rows, a.out);
  else
    hipLaunchKernelGGL((unpack_gather_kernel<false, kK>), dim3((unsigned)blocks), dim3(256), 0,
                       s, a.pool, a.pool_rows, a.physical, a.raw, a.lengths, a.ix, a.freqs,
                       a.freq_rows, a.out);
}

}  // namespace

extern "C" int rm_unpack_gather_bf16(const uint8_t* pool, int64_t pool_pages,
                                     const int32_t* physical, int64_t physical_stride_q,
                                     int64_t physical_stride_k, const int32_t* raw,
                                     int64_t raw_stride_q, int64_t raw_stride_k,
                                     const int32_t* lengths, int64_t length_stride,
                                     int64_t n_queries, int64_t selected_k, const float* freqs,
                                     int64_t freq_rows, uint16_t* out, void* stream) {
  return rm_unpack_gather_bf16_k(pool, pool_pages, RM_KEEP_COUNT, physical, physical_stride_q,
                                 physical_stride_k, raw, raw_stride_q, raw_stride_k, lengths,
                                 length_stride, n_queries, selected_k, freqs, freq_rows, out,
                                 stream);
}

extern "C" int rm_unpack_gather_bf16_k(const uint8_t* pool, int64_t pool_pages, int keep_count,
                                       const int32_t* physical, int64_t physical_stride_q,
                                       int64_t physical_stride_k, const int32_t* raw,
                                       int64_t raw_stride_q, int64_t raw_stride_k,
                                       const int32_t* lengths, int64_t length_stride,
                                       int64_t n_queries, int64_t selected_k,
                                       const float* freqs, int64_t freq_rows, uint16_t* out,
                                       void* stream) {
  if (n_queries < 0 || selected_k < 0 || pool_pages < 0 || freq_rows < 0) return RM_ERR_SHAPE;
  if (keep_count < 64 || keep_count > 448 || keep_count % 64) return RM_ERR_SHAPE;
  const int64_t total = n_queries * selected_k;
  if (total == 0) return RM_OK;
  if (!pool || !physical || !lengths || !out || (freqs && !raw)) return RM_ERR_NULL;
  if (!aligned(pool, 16) || !aligned(out, 16) || (freqs && !aligned(freqs, 16)))
    return RM_ERR_ALIGN;
  if (pool_pages > ((int64_t)1 << 25)) return RM_ERR_SHAPE;  // pool rows fit in int32
  int64_t blocks = (total + kWaves * kRows - 1) / (kWaves * kRows);
  if (blocks > 256 * 64) blocks = 256 * 64;
  Index ix;
  ix.ps_q = physical_stride_q;
  ix.ps_k = physical_stride_k;
  ix.rs_q = raw_stride_q;
  ix.rs_k = raw_stride_k;
  ix.ls = length_stride;
  ix.nk = selected_k;
  ix.total = total;
  ix.magic = 0;
  ix.shift = 0;
  // narrow indexing when every row index and element offset fits in int32
  auto span = [&](int64_t sq, int64_t sk) {
    return (n_queries - 1) * (sq < 0 ? -sq : sq) + (selected_k - 1) * (sk < 0 ? -sk : sk);
  };
  const int64_t lim = ((int64_t)1 << 31) - 1;
  const bool narrow = total <= lim && span(physical_stride_q, physical_stride_k) <= lim &&
                      span(length_stride, 0) <= lim &&
                      (!freqs || span(raw_stride_q, raw_stride_k) <= lim);
  if (narrow && selected_k > 1) {
    // round-up magic: l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1
    const uint64_t d = (uint64_t)selected_k;
    int l = 0;
    while (((uint64_t)1 << l) < d) ++l;
    ix.magic = (uint32_t)(((((uint64_t)1 << l) - d) << 32) / d + 1);
    ix.shift = (uint32_t)(l - 1);
  }
  hipStream_t s = (hipStream_t)stream;
  const Launch a{pool, pool_pages * kPageRecords, physical, raw, lengths, ix, freqs, freq_rows,
                 out};
  switch (keep_count) {
    case 64: launch_unpack<64>(narrow, blocks, a, s); break;
    case 128: launch_unpack<128>(narrow, blocks, a, s); break;
    case 192: launch_unpack<192>(narrow, blocks, a, s); break;
    case 256: launch_unpack<256>(narrow, blocks, a, s); break;
    case 320: launch_unpack<320>(narrow, blocks, a, s); break;
    case 384: launch_unpack<384>(narrow, blocks, a, s); break;
    default: launch_unpack<448>(narrow, blocks, a, s); break;
  }
  return hipGetLastError() == hipSuccess ? RM_OK : RM_ERR_LAUNCH;
}
