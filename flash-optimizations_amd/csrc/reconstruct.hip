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
constexpr int kRowsBulk = 4;   // rows per wave and loop iteration for large calls
constexpr int kSmallCall = 16384;  // below this many rows, one row per wave

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
  return u32x4{fp8_pair_to_bf16<false>(c03, scale), fp8_pair_to_bf16<true>(c03, scale),
               fp8_pair_to_bf16<false>(c47, scale), fp8_pair_to_bf16<true>(c47, scale)};
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

// Native 584-byte record of the lane-distributed BF16 row `o` (lane l holds
// coordinates 8l..8l+7) at workspace row `row` of a Native page layout: the
// seven NoPE groups re-encoded as UE8M0 scale + E4M3 codes from the row's own
// values (group amax over its 8 lanes; RNE(n / 2^e) by the scaled hardware
// conversion, equal to the software encode for every BF16 input with
// |n / 2^e| <= 448), the tail stored as is, scale row = 7 bytes + a zero pad.
__device__ __forceinline__ void store_native(uint8_t* out, int64_t row, u32x4 o, int lane) {
  uint8_t* const page = out + (row >> 6) * kNativePageBytes;
  uint8_t* const data = page + (row & 63) * kNativeDataBytes;
  uint32_t am = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t a = o[i] & 0x7fff7fffu;  // |lo|, |hi| as BF16 bits (order-preserving)
    am = max(am, max(a & 0xffffu, a >> 16));
  }
  am = max(am, (uint32_t)__shfl_xor((int)am, 1, 64));
  am = max(am, (uint32_t)__shfl_xor((int)am, 2, 64));
  am = max(am, (uint32_t)__shfl_xor((int)am, 4, 64));
  const int e = ue8m0_exponent(u2f(am << 16));
  if (lane < kNopeDim / 8) {
    const float scale = exp2i(e);
    // the BF16 pairs are rebuilt from their halves: a bit cast of a vector
    // element straight into the conversion's operand was compiled to read
    // element 0 for every pair
    bf16x2 p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      p[i] = bf16x2{__builtin_bit_cast(__bf16, (uint16_t)(o[i] & 0xffffu)),
                    __builtin_bit_cast(__bf16, (uint16_t)(o[i] >> 16))};
    s16x2 c01 = {0, 0}, c45 = {0, 0};
    c01 = fp8_pair<false>(c01, p[0], scale);
    c01 = fp8_pair<true>(c01, p[1], scale);
    c45 = fp8_pair<false>(c45, p[2], scale);
    c45 = fp8_pair<true>(c45, p[3], scale);
    *(u32x2*)(data + 8 * lane) = u32x2{__builtin_bit_cast(uint32_t, c01), __builtin_bit_cast(uint32_t, c45)};
  } else {
    *(u32x4*)(data + kNopeDim + 16 * (lane - kNopeDim / 8)) = o;
  }
  // scale row: the groups' exponents gathered into lane 56
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g) lo |= (uint32_t)(__builtin_amdgcn_readlane(e, 8 * g) + 127) << (8 * g);
#pragma unroll
  for (int g = 4; g < 7; ++g) hi |= (uint32_t)(__builtin_amdgcn_readlane(e, 8 * g) + 127) << (8 * (g - 4));
  if (lane == kNopeDim / 8)
    *(u32x2*)(page + kPageRecords * kNativeDataBytes + (row & 63) * kScaleBytes) = u32x2{lo, hi};
}

// kNative: write Native 584-byte records (the Adapter) instead of BF16 rows.
// kRows rows per wave and loop iteration: 4 for large calls (their loads
// overlap), 1 for small calls (four times the waves to hide latency with;
// 8,192 rows: 5.8 us instead of 7.1 us, while 35,840 rows run faster with 4).
// Large calls write their BF16 rows with non-temporal stores: at 16 MB and
// more the rows cannot stay in the L2 anyway, and streaming them keeps the
// caches for the records (35,840 rows: 9.3 us instead of 11.5 us; 1M rows:
// 0.271 ms instead of 0.286 ms, and the pack that follows in the bulk step
// 0.391 ms instead of 0.427 ms).
template <bool kNarrow, int kK, bool kNative, int kRows, bool kPlanes>
__global__ __launch_bounds__(256) void unpack_gather_kernel(
    PackedSrc src, int64_t pool_rows, const int32_t* __restrict__ physical,
    const int32_t* __restrict__ raw, const int32_t* __restrict__ lengths, Index ix,
    const float* __restrict__ freqs, int64_t freq_rows, void* __restrict__ out_) {
  uint16_t* const out = (uint16_t*)out_;
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
    const uint8_t* rec[kRows];   // this lane's 8-byte piece of the record
    const uint8_t* srec[kRows];  // bytes 512..519 (448 survivors: the scales)
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
      // contiguous pages hold 64 records each back to back: slot pp starts
      // pp * kBytes into the pool; planes: this lane's piece of each plane
      if (kPlanes) {
        rec[j] = lane < kK / 8 ? src.values + (uint64_t)pp * kK + 8 * lane
                 : lane < kK / 8 + 8 ? src.bitmaps + (uint64_t)pp * kBitmapBytes + 8 * (lane - kK / 8)
                                     : src.scales + (uint64_t)pp * kScaleBytes;
        srec[j] = src.scales + (uint64_t)pp * kScaleBytes;
      } else {
        rec[j] = src.values + (uint64_t)pp * kBytes + 8 * lane;
        srec[j] = src.values + (uint64_t)pp * kBytes + 512;
      }
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
      if (valid[j] && lane < kPieces) piece[j] = *(const u32x2*)rec[j];
      if (kBytes > 512 && valid[j]) extra[j] = *(const u32x2*)srec[j];
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
    for (int j = 0; j < kRows; ++j) {
      if (row0 + j >= ix.total) continue;
      if (kNative)
        store_native((uint8_t*)out_, row0 + j, o[j], lane);
      else if (kRows > 1)  // large calls: streaming stores, the rows outsize the caches
        __builtin_nontemporal_store(o[j], (u32x4*)(out + (row0 + j) * kHeadDim + 8 * lane));
      else
        *(u32x4*)(out + (row0 + j) * kHeadDim + 8 * lane) = o[j];
    }
  }
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

struct Launch {
  PackedSrc src;
  bool planes;
  int64_t pool_rows;
  const int32_t *physical, *raw, *lengths;
  Index ix;
  const float* freqs;
  int64_t freq_rows;
  void* out;
};

template <int kK, bool kNative, int kRows, bool kPlanes>
void launch_rows_layout(bool narrow, const Launch& a, hipStream_t s) {
  int64_t blocks = (a.ix.total + kWaves * kRows - 1) / (kWaves * kRows);
  if (blocks > 256 * 64) blocks = 256 * 64;
  if (narrow)
    hipLaunchKernelGGL((unpack_gather_kernel<true, kK, kNative, kRows, kPlanes>),
                       dim3((unsigned)blocks), dim3(256), 0, s, a.src, a.pool_rows, a.physical,
                       a.raw, a.lengths, a.ix, a.freqs, a.freq_rows, a.out);
  else
    hipLaunchKernelGGL((unpack_gather_kernel<false, kK, kNative, kRows, kPlanes>),
                       dim3((unsigned)blocks), dim3(256), 0, s, a.src, a.pool_rows, a.physical,
                       a.raw, a.lengths, a.ix, a.freqs, a.freq_rows, a.out);
}

template <int kK, bool kNative, int kRows>
void launch_rows(bool narrow, const Launch& a, hipStream_t s) {
  if (a.planes)
    launch_rows_layout<kK, kNative, kRows, true>(narrow, a, s);
  else
    launch_rows_layout<kK, kNative, kRows, false>(narrow, a, s);
}

template <int kK, bool kNative = false>
void launch_unpack(bool narrow, const Launch& a, hipStream_t s) {
  if (a.ix.total < kSmallCall)
    launch_rows<kK, kNative, 1>(narrow, a, s);
  else
    launch_rows<kK, kNative, kRowsBulk>(narrow, a, s);
}

// Argument checks and launch geometry shared by the reader entry points.
// Returns RM_OK with a.out == nullptr when there is nothing to launch.
// Contiguous pools are 16-byte aligned; each plane of a plane-layout pool is
// 8-byte aligned (its rows are multiples of 8 bytes).
int prepare(PackedSrc src, bool planes, int64_t pool_rows, const int32_t* physical, int64_t ps_q,
            int64_t ps_k, const int32_t* raw, int64_t rs_q, int64_t rs_k, const int32_t* lengths,
            int64_t ls, int64_t n_queries, int64_t selected_k, const float* freqs,
            int64_t freq_rows, void* out, Launch& a, bool& narrow) {
  a.out = nullptr;
  if (n_queries < 0 || selected_k < 0 || pool_rows < 0 || freq_rows < 0) return RM_ERR_SHAPE;
  const int64_t total = n_queries * selected_k;
  if (total == 0) return RM_OK;
  if (!src.values || (planes && (!src.bitmaps || !src.scales)) || !physical || !lengths ||
      !out || (freqs && !raw))
    return RM_ERR_NULL;
  if (!aligned(out, 16) || (freqs && !aligned(freqs, 16))) return RM_ERR_ALIGN;
  if (planes ? !(aligned(src.values, 8) && aligned(src.bitmaps, 8) && aligned(src.scales, 8))
             : !aligned(src.values, 16))
    return RM_ERR_ALIGN;
  if (pool_rows > ((int64_t)1 << 31)) return RM_ERR_SHAPE;  // pool rows fit in int32
  Index ix;
  ix.ps_q = ps_q;
  ix.ps_k = ps_k;
  ix.rs_q = rs_q;
  ix.rs_k = rs_k;
  ix.ls = ls;
  ix.nk = selected_k;
  ix.total = total;
  ix.magic = 0;
  ix.shift = 0;
  // narrow indexing when every row index and element offset fits in int32
  auto span = [&](int64_t sq, int64_t sk) {
    return (n_queries - 1) * (sq < 0 ? -sq : sq) + (selected_k - 1) * (sk < 0 ? -sk : sk);
  };
  const int64_t lim = ((int64_t)1 << 31) - 1;
  narrow = total <= lim && span(ps_q, ps_k) <= lim && span(ls, 0) <= lim &&
           (!freqs || span(rs_q, rs_k) <= lim);
  if (narrow && selected_k > 1) {
    // round-up magic: l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1
    const uint64_t d = (uint64_t)selected_k;
    int l = 0;
    while (((uint64_t)1 << l) < d) ++l;
    ix.magic = (uint32_t)(((((uint64_t)1 << l) - d) << 32) / d + 1);
    ix.shift = (uint32_t)(l - 1);
  }
  a = Launch{src, planes, pool_rows, physical, raw, lengths, ix, freqs, freq_rows, out};
  return RM_OK;
}

int launch_reader(PackedSrc src, bool planes, int64_t pool_rows, int keep_count,
                  const int32_t* physical, int64_t ps_q, int64_t ps_k, const int32_t* raw,
                  int64_t rs_q, int64_t rs_k, const int32_t* lengths, int64_t ls,
                  int64_t n_queries, int64_t selected_k, const float* freqs, int64_t freq_rows,
                  uint16_t* out, void* stream) {
  if (keep_count < 64 || keep_count > 448 || keep_count % 64) return RM_ERR_SHAPE;
  Launch a;
  bool narrow = false;
  const int st = prepare(src, planes, pool_rows, physical, ps_q, ps_k, raw, rs_q, rs_k, lengths,
                         ls, n_queries, selected_k, freqs, freq_rows, out, a, narrow);
  if (st != RM_OK || !a.out) return st;
  hipStream_t s = (hipStream_t)stream;
  switch (keep_count) {
    case 64: launch_unpack<64>(narrow, a, s); break;
    case 128: launch_unpack<128>(narrow, a, s); break;
    case 192: launch_unpack<192>(narrow, a, s); break;
    case 256: launch_unpack<256>(narrow, a, s); break;
    case 320: launch_unpack<320>(narrow, a, s); break;
    case 384: launch_unpack<384>(narrow, a, s); break;
    default: launch_unpack<448>(narrow, a, s); break;
  }
  return hipGetLastError() == hipSuccess ? RM_OK : RM_ERR_LAUNCH;
}

int launch_adapter(PackedSrc src, bool planes, int64_t pool_rows, const int32_t* physical,
                   int64_t ps_q, int64_t ps_k, const int32_t* raw, int64_t rs_q, int64_t rs_k,
                   const int32_t* lengths, int64_t ls, int64_t n_queries, int64_t selected_k,
                   const float* freqs, int64_t freq_rows, uint8_t* native, int64_t native_pages,
                   void* stream) {
  if (native_pages < 0 || n_queries < 0 || selected_k < 0) return RM_ERR_SHAPE;
  if (n_queries * selected_k > native_pages * kPageRecords) return RM_ERR_SHAPE;
  Launch a;
  bool narrow = false;
  const int st = prepare(src, planes, pool_rows, physical, ps_q, ps_k, raw, rs_q, rs_k, lengths,
                         ls, n_queries, selected_k, freqs, freq_rows, native, a, narrow);
  if (st != RM_OK || !a.out) return st;
  launch_unpack<kKeep, true>(narrow, a, (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? RM_OK : RM_ERR_LAUNCH;
}

PackedSrc contiguous(const uint8_t* pool) { return PackedSrc{pool, nullptr, nullptr}; }
PackedSrc plane_src(const uint8_t* values, const uint64_t* bitmaps, const uint8_t* scales) {
  return PackedSrc{values, (const uint8_t*)bitmaps, scales};
}
// Pool pages -> rows. A page count past the int32 slot range (or negative)
// maps to a row count that prepare() rejects.
int64_t page_rows(int64_t pool_pages) {
  if (pool_pages < 0) return -1;
  return pool_pages > ((int64_t)1 << 25) ? ((int64_t)1 << 32) : pool_pages * kPageRecords;
}

}  // namespace

extern "C" int rm_unpack_gather_bf16_k(const uint8_t* pool, int64_t pool_pages, int keep_count,
                                       const int32_t* physical, int64_t physical_stride_q,
                                       int64_t physical_stride_k, const int32_t* raw,
                                       int64_t raw_stride_q, int64_t raw_stride_k,
                                       const int32_t* lengths, int64_t length_stride,
                                       int64_t n_queries, int64_t selected_k,
                                       const float* freqs, int64_t freq_rows, uint16_t* out,
                                       void* stream) {
  return launch_reader(contiguous(pool), false, page_rows(pool_pages), keep_count, physical,
                       physical_stride_q, physical_stride_k, raw, raw_stride_q, raw_stride_k,
                       lengths, length_stride, n_queries, selected_k, freqs, freq_rows, out,
                       stream);
}

extern "C" int rm_unpack_gather_bf16_planes(const uint8_t* values, const uint64_t* bitmaps,
                                            const uint8_t* scales, int64_t rows, int keep_count,
                                            const int32_t* physical, int64_t physical_stride_q,
                                            int64_t physical_stride_k, const int32_t* raw,
                                            int64_t raw_stride_q, int64_t raw_stride_k,
                                            const int32_t* lengths, int64_t length_stride,
                                            int64_t n_queries, int64_t selected_k,
                                            const float* freqs, int64_t freq_rows, uint16_t* out,
                                            void* stream) {
  return launch_reader(plane_src(values, bitmaps, scales), true, rows, keep_count, physical,
                       physical_stride_q, physical_stride_k, raw, raw_stride_q, raw_stride_k,
                       lengths, length_stride, n_queries, selected_k, freqs, freq_rows, out,
                       stream);
}

extern "C" int rm_packed_to_native(const uint8_t* pool, int64_t pool_pages,
                                   const int32_t* physical, int64_t physical_stride_q,
                                   int64_t physical_stride_k, const int32_t* raw,
                                   int64_t raw_stride_q, int64_t raw_stride_k,
                                   const int32_t* lengths, int64_t length_stride,
                                   int64_t n_queries, int64_t selected_k, const float* freqs,
                                   int64_t freq_rows, uint8_t* native, int64_t native_pages,
                                   void* stream) {
  return launch_adapter(contiguous(pool), false, page_rows(pool_pages), physical,
                        physical_stride_q, physical_stride_k, raw, raw_stride_q, raw_stride_k,
                        lengths, length_stride, n_queries, selected_k, freqs, freq_rows, native,
                        native_pages, stream);
}

extern "C" int rm_packed_to_native_planes(const uint8_t* values, const uint64_t* bitmaps,
                                          const uint8_t* scales, int64_t rows,
                                          const int32_t* physical, int64_t physical_stride_q,
                                          int64_t physical_stride_k, const int32_t* raw,
                                          int64_t raw_stride_q, int64_t raw_stride_k,
                                          const int32_t* lengths, int64_t length_stride,
                                          int64_t n_queries, int64_t selected_k,
                                          const float* freqs, int64_t freq_rows, uint8_t* native,
                                          int64_t native_pages, void* stream) {
  return launch_adapter(plane_src(values, bitmaps, scales), true, rows, physical,
                        physical_stride_q, physical_stride_k, raw, raw_stride_q, raw_stride_k,
                        lengths, length_stride, n_queries, selected_k, freqs, freq_rows, native,
                        native_pages, stream);
}

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
