// Store kernels: Packed C4 record packer and the Native 584-byte control store.
//
// One wave64 per record; lane l owns coordinates 8l..8l+7 (16-byte BF16 or
// 32-byte FP32 loads, so a wave reads the 512-coordinate row in one coalesced
// sweep). No MFMA: the work is per-record selection, reductions and bit packing.
//
// Packed arithmetic (reference: training/losses.py:84-95, evaluate.py:65-91,
// test_integration.py:1588-1619; producer order in
// docs/agents/numerical-and-validation.md:22-26):
//   1. keep the K largest |x| (raw magnitudes; K = 256 by default, or a
//      survivor profile 64..448 in steps of 64); ties keep lower coordinates;
//   2. m = masked x; r = RN(1/RN(sqrt(sum(m^2)/512 + eps))), sum in the fixed
//      lane-then-pairwise-tree order; n = bf16(RN(RN(m*r)*w));
//   3. per 64-coordinate group: e = ceil(log2(max(amax|n|, 1e-4)/448)),
//      scale byte e + 127, code = e4m3_rne(n / 2^e);
//   4. codes of kept coordinates in ascending order, MSB-first bitmap words;
//      the record is K codes + 64 bitmap bytes + 8 scales (K + 72 bytes).
#include "remnant_device.h"
#include "remnant_mi355x.h"

using namespace rm;

namespace {

constexpr int kWaves = 4;

// Geometry of a K-survivor Packed record (K = kKeep gives the 328-byte default).
template <int kK>
struct Rec {
  static constexpr int kBytes = kK + kBitmapBytes + kScaleBytes;  // K + 72
  static constexpr int kPage = kPageRecords * kBytes;
  static constexpr int kPieces = kBytes / 8;                        // 8-byte stores
  static constexpr int kSpill = (kBytes + 15) / 16 * 16;  // 64 scratch bytes after it
  static_assert(kK % 64 == 0 && kK >= 64 && kK <= 448, "survivor profiles are 64..448");
};

template <bool kBf16>
__device__ __forceinline__ void load_row8(const void* x, int64_t row, int64_t stride,
                                          int lane, float* v) {
  if (kBf16) {
    const uint16_t* p = (const uint16_t*)x + row * stride + 8 * lane;
    u32x4 d = *(const u32x4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = u2f(d[i] << 16);
      v[2 * i + 1] = u2f(d[i] & 0xffff0000u);
    }
  } else {
    const float* p = (const float*)x + row * stride + 8 * lane;
    f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
}

// The lane's raw slice of a row (BF16: one 16-byte load; FP32: two), loaded
// one record ahead of its use so the load latency overlaps the previous
// record's work. kStream (large calls): rows are read once, so streaming
// (non-temporal) loads leave the caches to the scattered record writes.
struct RowRaw {
  u32x4 a, b;
};

template <bool kStream>
__device__ __forceinline__ u32x4 load16(const u32x4* p) {
  if constexpr (kStream) return __builtin_nontemporal_load(p);
  return *p;
}
template <bool kBf16, bool kStream>
__device__ __forceinline__ RowRaw load_raw(const void* x, int64_t row, int64_t stride, int lane) {
  RowRaw r;
  if (kBf16) {
    r.a = load16<kStream>((const u32x4*)((const uint16_t*)x + row * stride + 8 * lane));
    r.b = r.a;
  } else {
    const float* p = (const float*)x + row * stride + 8 * lane;
    r.a = load16<kStream>((const u32x4*)p);
    r.b = load16<kStream>((const u32x4*)(p + 4));
  }
  return r;
}
// One 8-byte piece of a record (kStream: a streaming store).
template <bool kStream>
__device__ __forceinline__ void store8(u32x2 v, u32x2* dst) {
  if constexpr (kStream) {
    __builtin_nontemporal_store(v, dst);
  } else {
    *dst = v;
  }
}

template <bool kBf16>
__device__ __forceinline__ void unpack_raw(const RowRaw& r, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (kBf16) {
      v[2 * i] = u2f(r.a[i] << 16);
      v[2 * i + 1] = u2f(r.a[i] & 0xffff0000u);
    } else {
      v[i] = u2f(r.a[i]);
      v[4 + i] = u2f(r.b[i]);
    }
  }
}

// Lane exchanges within rows of 16 (DPP): xor 1 and xor 2 inside quads, then
// the mirrors, which pair each lane with one in the other half of its group of
// 8 (16). In a butterfly reduction every lane of an aligned group already holds
// the same value, so any partner in the other half gives the xor-partner's value.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within 16

template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_value(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

// Sum over the wave in the fixed pairwise order (distance 1, 2, ..., 32):
// level d adds the value of lane l ^ d. Addition commutes bitwise, so the
// butterfly below yields exactly that result in every lane.
__device__ __forceinline__ float wave_tree_sum(float p) {
  p = p + dpp<kDppXor1>(p);
  p = p + dpp<kDppXor2>(p);
  p = p + dpp<kDppHalfMirror>(p);
  p = p + dpp<kDppMirror>(p);
  // rows of 16 are now uniform (r0..r3): row broadcast 15 gives rows 1 and 3
  // r0 + r1 and r2 + r3, row broadcast 31 gives row 3 (r0 + r1) + (r2 + r3)
  p = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(p), 0x142, 0xa, 0xf, false)) + p;
  p = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(p), 0x143, 0xc, 0xf, false)) + p;
  return lane_value(p, 63);
}

__device__ __forceinline__ int popc_ballot(bool pred) {
  return __popcll(__ballot(pred));
}


// Inclusive prefix sum of x over the wave's lanes (row shifts within rows of
// 16, then row broadcasts 15 and 31); the exclusive sum subtracts x.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
  int v = x;
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false); // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false); // row_bcast:31
  return v;
}
__device__ __forceinline__ int wave_exclusive_sum(int x) { return wave_inclusive_sum(x) - x; }

// Exclusive count of set predicates in lanes below this one.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// #{key >= c} over the wave's 512 keys (one ballot per key slot, popcounts
// on the scalar unit).
__device__ __forceinline__ int count_ge(const uint32_t* key, uint32_t c) {
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) cnt += popc_ballot(key[i] >= c);
  return cnt;
}

// Bit-serial radix select of the kK-th largest key below an established
// prefix: bits kTop..kLow, fully unrolled. `prefix` holds the threshold's bits
// above kTop and `at` = #{key >= prefix}; on return `prefix` is the threshold
// and `at` the count at the last accepted step.
template <int kTop, int kLow, int kK>
__device__ __forceinline__ void radix_bits(const uint32_t* key, uint32_t& prefix, int& at) {
#pragma unroll
  for (int b = kTop; b >= kLow; --b) {
    const uint32_t cand = prefix | (1u << b);
    const int cnt = count_ge(key, cand);
    const bool take = cnt >= kK;
    prefix = take ? cand : prefix;
    at = take ? cnt : at;
  }
}

// Seven more bits of the threshold from a histogram instead of seven
// bit-serial counts. The threshold lies in [base, base + 128 << kShift); keys
// in that range fall into bin (key - base) >> kShift. Keys are magnitudes:
// BF16 keys the 15-bit pattern (one level over the binade: base = E << 7,
// kShift = 0), FP32 keys the 31-bit one (levels with kShift = 16, 9, 2 below
// base = E << 23, then two bit-serial steps). The wave's 128 LDS bins (zero on
// entry, zero again on return) count the range's keys; lane l reads bins
// 127 - 2l and 126 - 2l, so an inclusive scan over the lanes gives S(m) =
// #{range keys in bins >= m}, and lane 63 holds S(0), the range's keys.
struct BinScan {
  int incl;   // S(126 - 2 lane)
  int lo;     // bin 126 - 2 lane
  int hi;     // bin 127 - 2 lane
  int total;  // S(0)
};
template <int kShift>
__device__ __forceinline__ BinScan bin_scan(const uint32_t* key, uint32_t base, uint32_t* hist) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t idx = key[i] - base;
    if (idx < (128u << kShift))
      __hip_atomic_fetch_add(hist + (idx >> kShift), 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WAVEFRONT);
  }
  wave_lds_sync();
  const int lane = wave_lane();
  uint64_t* const pair = (uint64_t*)(hist + 126 - 2 * lane);
  const uint64_t h = *pair;
  *pair = 0;  // in order after the read: the bins are clear for the next range
  BinScan b;
  b.lo = (int)(uint32_t)h;
  b.hi = (int)(uint32_t)(h >> 32);
  b.incl = wave_inclusive_sum(b.lo + b.hi);
  b.total = __builtin_amdgcn_readlane(b.incl, 63);
  return b;
}
// The threshold's bin from a scan whose range holds it: `above` = #{key >= base
// + (128 << kShift)} < kK <= above + S(0). The bin is the largest m with above
// + S(m) >= kK. On return `prefix` = base + (m << kShift), `at` = #{key >=
// prefix}, as the bit-serial search leaves them, and `tied` = the bin's count
// (for BF16 keys, the keys equal to the threshold; otherwise the next level's
// range).
template <int kK, int kShift>
__device__ __forceinline__ void bin_pick(const BinScan& b, uint32_t base, int above,
                                         uint32_t& prefix, int& at, int& tied) {
  const int need = kK - above;  // >= 1, and S(0) >= need
  const int l = (int)__builtin_ctzll(__ballot(b.incl >= need));
  const int s_lo = __builtin_amdgcn_readlane(b.incl, l);       // S(126 - 2l)
  const int s_hi = s_lo - __builtin_amdgcn_readlane(b.lo, l);  // S(127 - 2l)
  const bool upper = s_hi >= need;
  prefix = base + ((uint32_t)(upper ? 127 - 2 * l : 126 - 2 * l) << kShift);
  at = above + (upper ? s_hi : s_lo);
  tied = upper ? __builtin_amdgcn_readlane(b.hi, l) : __builtin_amdgcn_readlane(b.lo, l);
}
template <int kK, int kShift>
__device__ __forceinline__ void bin_histogram(const uint32_t* key, uint32_t base, int above,
                                              uint32_t* hist, uint32_t& prefix, int& at,
                                              int& tied) {
  bin_pick<kK, kShift>(bin_scan<kShift>(key, base, hist), base, above, prefix, at, tied);
}

// Masked values: m[i] = v[i] where bit i of `keep` is set, else 0.
__device__ __forceinline__ void mask_by_keep(const float* v, uint32_t keep, float* m) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
    m[i] = __int_as_float(__float_as_int(v[i]) & __builtin_amdgcn_sbfe((int)keep, i, 1));
}

// Keep mask for BF16 keys at threshold t with at = #{key >= t} and tied =
// #{key == t}: every key above t, and the (kK - (at - tied)) lowest-coordinate
// keys equal to t; m receives the kept values. Keys and t are below 2^31, so
// key < t is the borrow (and the sign) of key - t, which also clears the
// pruned value, and key > t is the sign of t - key; the sign bits are shifted
// into the byte by a funnel shift, slot 7 first. Ties are ranked by a wave
// prefix sum of each lane's tie count; a lane keeps its first `admit` ties,
// cut at the position of its admit-th tie (byte `admit` of the selector table
// entry of its tie byte).
template <int kK>
__device__ __forceinline__ uint32_t keep_at_threshold(const uint32_t* key, const float* v,
                                                      float* m, uint32_t t, int at, int tied,
                                                      const uint64_t* ctab) {
  uint32_t lt = 0;
  bool below[8];
#pragma unroll
  for (int i = 7; i >= 0; --i) {
    uint32_t borrow;
    const uint32_t x = __builtin_subc(key[i], t, 0u, &borrow);
    lt = __builtin_amdgcn_alignbit(lt, x, 31);
    below[i] = borrow != 0;
  }
  const uint32_t ge = ~lt & 0xffu;
  if (at == kK) {
#pragma unroll
    for (int i = 0; i < 8; ++i) m[i] = below[i] ? 0.0f : v[i];
    return ge;
  }
  uint32_t gt = 0;
#pragma unroll
  for (int i = 7; i >= 0; --i) gt = __builtin_amdgcn_alignbit(gt, t - key[i], 31);
  gt &= 0xffu;
  const uint32_t tie = ge & ~gt;
  const int need = kK - (at - tied);  // ties to admit: 1 <= need < tied
  const int cnt = __popc(tie);
  const int admit = min(max(need - wave_exclusive_sum(cnt), 0), cnt);
  const uint32_t cut = (uint32_t)(ctab[tie] >> (8 * (admit & 7))) & 7u;
  const uint32_t keep = gt | (admit < cnt ? tie & ((1u << cut) - 1u) : tie);
  mask_by_keep(v, keep, m);
  return keep;
}

// Keep mask (bit i = coordinate 8*lane + i) of the kK largest magnitudes.
// The threshold (the kK-th largest key) is found exponent first: the previous
// record's threshold exponent `hint` and its neighbours are tried
// (consecutive records of a layer have thresholds within a binade or two).
// One count at the start of the hint's binade, then the histogram of that
// binade, whose total gives the count at its end; a second count tries the
// binade below or above. The threshold binade's histogram
// gives the top seven mantissa bits (FP32 keys: up to two more histogram
// levels and two bit-serial steps for the bits below, ending at the first
// level whose bin holds exactly the keys still needed); when the exponent is
// none of the three the search runs bit-serially over all key bits. Both ways
// give the same keep set. `at` is the count at the last accepted step, i.e.
// #{key >= threshold}; only when it exceeds kK is there a boundary tie to
// admit in coordinate order.
template <bool kBf16, int kK>
__device__ __forceinline__ uint32_t select_top(const uint32_t* key, const float* v, float* m,
                                               uint32_t& hint, uint32_t* hist,
                                               const uint64_t* ctab) {
  constexpr int kExp = kBf16 ? 7 : 23;     // key bit of the exponent's LSB
  constexpr int kLevel = kBf16 ? 0 : 16;   // bin width (log2) of the binade's histogram
  const uint32_t e = hint;                 // 1 <= e <= 252
  uint32_t prefix = 0, te = 0;
  int at = 512, tied = 0;
  bool found = false;
  // The binade of `hint` first: one count at its start, and its histogram,
  // whose total gives the count at its end. (Each histogram is picked where
  // it is scanned: its per-lane scan values then need no merging.)
  const int c_e = count_ge(key, e << kExp);
  int c_up = -1;
  if (c_e >= kK) {
    const BinScan b = bin_scan<kLevel>(key, e << kExp, hist);
    c_up = c_e - b.total;
    if (c_up < kK) {
      te = e;
      found = true;
      bin_pick<kK, kLevel>(b, e << kExp, c_up, prefix, at, tied);
    }
  }
  if (!found) {  // the binade below or above it
    int above = 0;
    if (c_up < 0) {
      if (count_ge(key, (e - 1) << kExp) >= kK) {
        te = e - 1;
        above = c_e;
        found = true;
      }
    } else {
      const int c_up2 = count_ge(key, (e + 2) << kExp);
      if (c_up2 < kK) {
        te = e + 1;
        above = c_up2;
        found = true;
      }
    }
    if (found)
      bin_pick<kK, kLevel>(bin_scan<kLevel>(key, te << kExp, hist), te << kExp, above, prefix, at,
                           tied);
  }
  if (found) {
    if (kBf16) {
      hint = te < 1 ? 1u : (te > 252 ? 252u : te);
      return keep_at_threshold<kK>(key, v, m, prefix, at, tied, ctab);
    }
    // A level whose threshold bin holds exactly the keys still needed (at ==
    // kK: the keys at or above the bin's start are the kK largest, the next
    // key lies below the bin) ends the search: the finer levels would move
    // the prefix up to the kK-th largest key and leave the same keep set.
    if (at != kK) {
      bin_histogram<kK, 9>(key, prefix, at - tied, hist, prefix, at, tied);
      if (at != kK) {
        bin_histogram<kK, 2>(key, prefix, at - tied, hist, prefix, at, tied);
        if (at != kK) radix_bits<1, 0, kK>(key, prefix, at);
      }
    }
  } else {
    prefix = 0;
    at = 512;
    radix_bits<kExp + 7, 0, kK>(key, prefix, at);
  }
  te = prefix >> kExp;
  hint = te < 1 ? 1u : (te > 252 ? 252u : te);
  uint32_t keep = 0;
  if (at == kK) {
#pragma unroll
    for (int i = 0; i < 8; ++i) keep |= (key[i] >= prefix ? 1u : 0u) << i;
    mask_by_keep(v, keep, m);
    return keep;
  }
  // admit the (kK - #{key > prefix}) lowest-coordinate ties at the threshold
  int gt = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) gt += popc_ballot(key[i] > prefix);
  const int need = kK - gt;
  int before = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) before += lanes_below(__ballot(key[i] == prefix));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool tie = key[i] == prefix;
    const bool k = key[i] > prefix || (tie && before < need);
    before += tie ? 1 : 0;
    keep |= (k ? 1u : 0u) << i;
  }
  mask_by_keep(v, keep, m);
  return keep;
}

// Rows rec, rec + step, ... below end of this wave. Runs: the n rows cut into
// contiguous runs of ceil(n / waves) over the grid's waves (one row per wave
// when n is small; consecutive rows are read and prefetched from the same DRAM
// neighbourhood). Otherwise a grid stride.
__device__ __forceinline__ void wave_rows(bool runs, int64_t n, int wave, int64_t& rec,
                                          int64_t& end, int64_t& step) {
  const int64_t waves = (int64_t)gridDim.x * kWaves;
  const int64_t id = (int64_t)blockIdx.x * kWaves + wave;
  if (runs) {
    const int64_t per = (n + waves - 1) / waves;
    rec = id * per;
    end = rec + per < n ? rec + per : n;
    step = 1;
  } else {
    rec = id;
    end = n;
    step = waves;
  }
}

template <bool kBf16, int kK, bool kPlanes, bool kStream>
__global__ __launch_bounds__(256) void pack_rows_kernel(
    const void* __restrict__ x, int64_t stride, const float* __restrict__ weight, float eps,
    const int32_t* __restrict__ slots, int64_t n, PackedDst dst_pool, int64_t pool_rows) {
  using R = Rec<kK>;
  __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][R::kSpill + 64];
  // compaction selectors: for a keep byte, byte p of the entry is the slot
  // (0..7) of its p-th survivor, or 0x0c (a zero byte) past the last one
  __shared__ uint64_t ctab[256];
  // per-wave histogram bins of the threshold binade's mantissas (kept zero
  // between records)
  __shared__ __attribute__((aligned(16))) uint32_t bins[kWaves][128];
  const int lane = wave_lane();
  const int wave = uniform((int)(threadIdx.x >> 6));
  // BF16 rows (1 KB): a contiguous run per wave (measured 3.7 % faster on the
  // 1M-row bulk pack); FP32 rows (2 KB): the grid stride (1 % faster). The
  // first row, its slot and the weights are requested before the LDS tables
  // are built, so their latency covers that set-up (small calls: the decode
  // store's few rows).
  int64_t rec, end, step;
  wave_rows(kBf16, n, wave, rec, end, step);
  RowRaw cur{};
  int32_t cur_slot = -1;
  if (rec < end) {
    cur = load_raw<kBf16, kStream>(x, rec, stride, lane);
    cur_slot = slots[rec];
  }
  float w[8];
  {
    f32x4 a = *(const f32x4*)(weight + 8 * lane), b = *(const f32x4*)(weight + 8 * lane + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = a[i];
      w[4 + i] = b[i];
    }
  }
  bins[threadIdx.x >> 6][2 * (threadIdx.x & 63)] = 0;
  bins[threadIdx.x >> 6][2 * (threadIdx.x & 63) + 1] = 0;
  {
    const uint32_t k = threadIdx.x;  // 256 threads: one entry each
    uint64_t sel = 0x0c0c0c0c0c0c0c0cull;
    int p = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if ((k >> i) & 1u) {
        sel = (sel & ~(0xffull << (8 * p))) | ((uint64_t)i << (8 * p));
        ++p;
      }
    }
    ctab[k] = sel;
  }
  __syncthreads();
  uint8_t* st = stage[wave];
  uint32_t hint = 126;  // threshold exponent of this wave's previous record (|x| ~ 2^-1)
  for (; rec < end; rec += step) {
    // the next record's row and slot are in flight while this one is packed
    const RowRaw raw = cur;
    const int32_t slot = cur_slot;
    if (rec + step < end) {
      cur = load_raw<kBf16, kStream>(x, rec + step, stride, lane);
      cur_slot = slots[rec + step];
    }
    if (slot < 0 || slot >= pool_rows) continue;
    float v[8];
    uint32_t key[8];
    unpack_raw<kBf16>(raw, v);
#pragma unroll
    for (int i = 0; i < 8; ++i)  // BF16: the 15-bit magnitude; FP32: the 31-bit one
      key[i] = kBf16 ? (raw.a[i / 2] >> (16 * (i & 1))) & 0x7fffu : f2u(v[i]) & 0x7fffffffu;
    // keep mask and the kept values m (pruned values cleared)
    float m[8];
    const uint32_t keep = select_top<kBf16, kK>(key, v, m, hint, bins[wave], ctab);

    // masked RMSNorm
    float p = m[0] * m[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) {
      float sq = m[i] * m[i];
      p = p + sq;
    }
    const float sumsq = wave_tree_sum(p);
    const float r = inv_rms(sumsq, eps);
    // n = bf16(RN(RN(m * r) * w)) with the hardware round-to-nearest-even
    // conversion (identical to the software rounding for every non-NaN input)
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      y[i] = m[i] * r;
      y[i] = y[i] * w[i];
    }
    bf16x2 nb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) nb[i] = bf16_pair(y[2 * i], y[2 * i + 1]);
    // group amax: rounding is monotonic, so max |bf16(y)| = bf16(max |y|)
    float ay = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
    ay = fmaxf(ay, fmaxf(fmaxf(fabsf(y[4]), fabsf(y[5])), fmaxf(fabsf(y[6]), fabsf(y[7]))));
    // max over the 8 lanes of the group, on the bit patterns (ay >= 0, so
    // integer order is float order): one DPP max per level
    int ai = __float_as_int(ay);
    ai = max(ai, __builtin_amdgcn_update_dpp(0, ai, kDppXor1, 0xf, 0xf, false));
    ai = max(ai, __builtin_amdgcn_update_dpp(0, ai, kDppXor2, 0xf, 0xf, false));
    ai = max(ai, __builtin_amdgcn_update_dpp(0, ai, kDppHalfMirror, 0xf, 0xf, false));
    const float amax = (float)(__bf16)__int_as_float(ai);
    const int e = ue8m0_exponent(amax);

    // E4M3 codes = RNE(n / 2^e) by the scaled hardware conversion (identical to
    // the software encode for every in-range BF16 input); |n / 2^e| <= 448
    const float scale = exp2i(e);
    s16x2 c01 = {0, 0}, c45 = {0, 0};
    c01 = fp8_pair<false>(c01, nb[0], scale);
    c01 = fp8_pair<true>(c01, nb[1], scale);
    c45 = fp8_pair<false>(c45, nb[2], scale);
    c45 = fp8_pair<true>(c45, nb[3], scale);
    const uint32_t lo = __builtin_bit_cast(uint32_t, c01), hi = __builtin_bit_cast(uint32_t, c45);

    // compaction: survivors go to [rank, rank + popcount) in coordinate order,
    // rank = survivors in lower lanes (a wave prefix sum). v_perm packs the
    // lane's surviving codes into the low bytes of 8 (zeros above), which are
    // OR-ed into the zeroed code area at byte offset rank: two 8-byte LDS ORs
    // at the aligned words the run touches (neighbouring lanes share words).
    const int cnt = __popc(keep);
    const int rank = wave_exclusive_sum(cnt);
    if (lane < kK / 8) *(uint64_t*)(st + 8 * lane) = 0;
    const uint64_t sel = ctab[keep];
    const uint64_t run = ((uint64_t)__builtin_amdgcn_perm(hi, lo, (uint32_t)(sel >> 32)) << 32) |
                         __builtin_amdgcn_perm(hi, lo, (uint32_t)sel);
    const uint32_t sh = 8u * (uint32_t)(rank & 7);
    uint64_t* const word = (uint64_t*)(st + (rank & ~7));
    __hip_atomic_fetch_or(word, run << sh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
    __hip_atomic_fetch_or(word + 1, (run >> 1) >> (63u - sh), __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_WAVEFRONT);
    // bitmap byte: coordinate 8l+i is bit 7-i of byte 7 - l%8 of word l/8
    const uint32_t rev = __builtin_bitreverse32(keep) >> 24;
    st[kK + 8 * (lane >> 3) + 7 - (lane & 7)] = (uint8_t)rev;
    if ((lane & 7) == 0) st[kK + kBitmapBytes + (lane >> 3)] = (uint8_t)(e + 127);
    wave_lds_sync();

    // the record is 8-byte aligned: one 8-byte store per lane (41 lanes for the
    // 328-byte record; the 520-byte 448-survivor record needs a 65th piece).
    // Contiguous pages hold 64 records back to back (slot s at s * kBytes);
    // planes take lane pieces 0..K/8-1 (codes), the next 8 (bitmap) and the
    // one after them (scales) at row `slot` of their plane. Streaming stores
    // on large calls: a record shares its first and last 128-byte lines with
    // records that other waves write at unrelated times (1M-row bulk pack with
    // random slots: 0.418 -> 0.400 ms together with the streaming row loads).
    // Smaller calls, whose rows and records stay in the caches, are faster
    // with ordinary loads and stores.
    if (kPlanes) {
      uint8_t* dst = lane < kK / 8 ? dst_pool.values + (int64_t)slot * kK + 8 * lane
                     : lane < kK / 8 + 8
                         ? dst_pool.bitmaps + (int64_t)slot * kBitmapBytes + 8 * (lane - kK / 8)
                         : dst_pool.scales + (int64_t)slot * kScaleBytes;
      if (lane < R::kPieces) store8<kStream>(*(const u32x2*)(st + 8 * lane), (u32x2*)dst);
      if (R::kPieces > 64 && lane == 0)
        store8<kStream>(*(const u32x2*)(st + 512),
                        (u32x2*)(dst_pool.scales + (int64_t)slot * kScaleBytes));
    } else {
      uint8_t* dst = dst_pool.values + (int64_t)slot * R::kBytes;
      if (lane < R::kPieces)
        store8<kStream>(*(const u32x2*)(st + 8 * lane), (u32x2*)(dst + 8 * lane));
      if (R::kPieces > 64 && lane < R::kPieces - 64)
        store8<kStream>(*(const u32x2*)(st + 512 + 8 * lane), (u32x2*)(dst + 512 + 8 * lane));
    }
    wave_lds_sync();
  }
}

template <bool kBf16>
__global__ __launch_bounds__(256) void native_store_kernel(
    const void* __restrict__ x, int64_t stride, const float* __restrict__ weight, float eps,
    const int32_t* __restrict__ slots, const int32_t* __restrict__ position,
    const float* __restrict__ freqs, int64_t freq_rows, int64_t n, uint8_t* __restrict__ pool,
    int64_t pool_rows) {
  const int lane = wave_lane();
  const int wave = uniform((int)(threadIdx.x >> 6));
  float w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = weight[8 * lane + i];
  int64_t rec0, end, step;
  wave_rows(kBf16, n, wave, rec0, end, step);
  for (int64_t rec = rec0; rec < end; rec += step) {
    const int64_t slot = slots[rec];
    if (slot < 0 || slot >= pool_rows) continue;
    int64_t pos = 0;
    if (freqs) {
      pos = position[rec];
      if (pos < 0 || pos * 4 >= freq_rows) continue;
    }
    float v[8];
    load_row8<kBf16>(x, rec, stride, lane, v);
    float p = v[0] * v[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) {
      float sq = v[i] * v[i];
      p = p + sq;
    }
    const float sumsq = wave_tree_sum(p);
    const float r = inv_rms(sumsq, eps);
    float nf[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float y = v[i] * r;
      y = y * w[i];
      nf[i] = bf16_to_f32(bf16_rne(y));
      amax = fmaxf(amax, fabsf(nf[i]));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    uint8_t* page = pool + (slot >> 6) * kNativePageBytes;
    const int row = (int)(slot & 63);
    uint8_t* data = page + row * kNativeDataBytes;
    if (lane < kNopeDim / 8) {
      const int e = ue8m0_exponent(amax);
      const float inv = exp2i(-e);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo |= e4m3_rne(nf[i] * inv) << (8 * i);
        hi |= e4m3_rne(nf[4 + i] * inv) << (8 * i);
      }
      *(u32x2*)(data + 8 * lane) = u32x2{lo, hi};
      uint8_t* srow = page + kPageRecords * kNativeDataBytes + row * kScaleBytes;
      if ((lane & 7) == 0) srow[lane >> 3] = (uint8_t)(e + 127);
      if (lane == 0) srow[7] = 0;
    } else {
      if (freqs) {
        const float* f = freqs + (pos * 4) * (2 * kRopePairs) + 8 * (lane - kNopeDim / 8);
        float cs[8];
        f32x4 a = *(const f32x4*)f, b = *(const f32x4*)(f + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          cs[i] = a[i];
          cs[4 + i] = b[i];
        }
        rope4(nf, cs);
      }
      u32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = bf16_rne(nf[2 * i]) | (bf16_rne(nf[2 * i + 1]) << 16);
      *(u32x4*)(data + kNopeDim + 16 * (lane - kNopeDim / 8)) = o;
    }
  }
}

int grid_for(int64_t n) {
  int64_t blocks = (n + kWaves - 1) / kWaves;
  // 256 CUs x 64 blocks (256 waves per CU over the launch): measured on the
  // 1M-row bulk pack against 32, 128 and 256 blocks per CU, this one is fastest
  const int64_t cap = 256 * 64;
  return (int)(blocks < cap ? blocks : cap);
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

struct PackLaunch {
  bool bf16, planes;
  const void* x;
  int64_t stride;
  const float* weight;
  float eps;
  const int32_t* slots;
  int64_t n;
  PackedDst pool;
  int64_t rows;
  hipStream_t stream;
};

template <int kK, bool kPlanes, bool kStream>
void launch_pack_mode(const PackLaunch& L) {
  if (L.bf16)
    hipLaunchKernelGGL((pack_rows_kernel<true, kK, kPlanes, kStream>), dim3(grid_for(L.n)),
                       dim3(256), 0, L.stream, L.x, L.stride, L.weight, L.eps, L.slots, L.n,
                       L.pool, L.rows);
  else
    hipLaunchKernelGGL((pack_rows_kernel<false, kK, kPlanes, kStream>), dim3(grid_for(L.n)),
                       dim3(256), 0, L.stream, L.x, L.stride, L.weight, L.eps, L.slots, L.n,
                       L.pool, L.rows);
}

// Streaming row loads and record stores above this many rows. Measured with
// random slots (paired rounds, both input types): ordinary accesses are 4-8 %
// faster from 24 to 131,072 rows (R128 3.62 -> 3.33 us, 131,072 BF16 rows 62.8
// -> 61.5 us); streaming ones 3 % (BF16) and 14 % (FP32) faster at 1M rows.
constexpr int64_t kStreamRows = 131072;

template <int kK, bool kPlanes>
void launch_pack_layout(const PackLaunch& L) {
  if (L.n > kStreamRows)
    launch_pack_mode<kK, kPlanes, true>(L);
  else
    launch_pack_mode<kK, kPlanes, false>(L);
}

template <int kK>
void launch_pack(const PackLaunch& L) {
  if (L.planes)
    launch_pack_layout<kK, true>(L);
  else
    launch_pack_layout<kK, false>(L);
}

// Argument checks and launch shared by the store entry points. Contiguous
// pools are 16-byte aligned, planes 8-byte aligned.
int pack_any(const void* x, int x_dtype, int64_t x_row_stride, const float* weight, float eps,
             const int32_t* dst_slot, int64_t n, PackedDst pool, bool planes, int64_t rows,
             int keep_count, void* stream) {
  if (n < 0 || rows < 0) return RM_ERR_SHAPE;
  if (keep_count < 64 || keep_count > 448 || keep_count % 64) return RM_ERR_SHAPE;
  if (n == 0) return RM_OK;
  if (!x || !weight || !dst_slot || !pool.values || (planes && (!pool.bitmaps || !pool.scales)))
    return RM_ERR_NULL;
  if (x_dtype != RM_F32 && x_dtype != RM_BF16) return RM_ERR_DTYPE;
  if (x_row_stride < kHeadDim && n > 1) return RM_ERR_SHAPE;
  const int esize = x_dtype == RM_BF16 ? 2 : 4;
  if (!aligned(x, 16) || ((x_row_stride * esize) & 15) || !aligned(weight, 16))
    return RM_ERR_ALIGN;
  if (planes ? !(aligned(pool.values, 8) && aligned(pool.bitmaps, 8) && aligned(pool.scales, 8))
             : !aligned(pool.values, 16))
    return RM_ERR_ALIGN;
  const PackLaunch L{x_dtype == RM_BF16, planes, x, x_row_stride, weight, eps, dst_slot, n,
                     pool, rows, (hipStream_t)stream};
  switch (keep_count) {
    case 64: launch_pack<64>(L); break;
    case 128: launch_pack<128>(L); break;
    case 192: launch_pack<192>(L); break;
    case 256: launch_pack<256>(L); break;
    case 320: launch_pack<320>(L); break;
    case 384: launch_pack<384>(L); break;
    default: launch_pack<448>(L); break;
  }
  return hipGetLastError() == hipSuccess ? RM_OK : RM_ERR_LAUNCH;
}

}  // namespace

extern "C" int rm_pack_rows(const void* x, int x_dtype, int64_t x_row_stride,
                            const float* weight, float eps, const int32_t* dst_slot, int64_t n,
                            uint8_t* pool, int64_t pool_pages, void* stream) {
  return rm_pack_rows_k(x, x_dtype, x_row_stride, weight, eps, dst_slot, n, pool, pool_pages,
                        RM_KEEP_COUNT, stream);
}

extern "C" int rm_pack_rows_k(const void* x, int x_dtype, int64_t x_row_stride,
                              const float* weight, float eps, const int32_t* dst_slot,
                              int64_t n, uint8_t* pool, int64_t pool_pages, int keep_count,
                              void* stream) {
  if (pool_pages < 0 || pool_pages > ((int64_t)1 << 25)) return RM_ERR_SHAPE;  // int32 slots
  return pack_any(x, x_dtype, x_row_stride, weight, eps, dst_slot, n,
                  PackedDst{pool, nullptr, nullptr}, false, pool_pages * kPageRecords,
                  keep_count, stream);
}

extern "C" int rm_pack_rows_planes(const void* x, int x_dtype, int64_t x_row_stride,
                                   const float* weight, float eps, const int32_t* dst_slot,
                                   int64_t n, uint8_t* values, uint64_t* bitmaps,
                                   uint8_t* scales, int64_t rows, int keep_count, void* stream) {
  if (rows > ((int64_t)1 << 31)) return RM_ERR_SHAPE;  // int32 slots
  return pack_any(x, x_dtype, x_row_stride, weight, eps, dst_slot, n,
                  PackedDst{values, (uint8_t*)bitmaps, scales}, true, rows, keep_count, stream);
}

extern "C" int rm_native_store_rows(const void* x, int x_dtype, int64_t x_row_stride,
                                    const float* weight, float eps, const int32_t* dst_slot,
                                    const int32_t* position, const float* freqs,
                                    int64_t freq_rows, int64_t n, uint8_t* pool,
                                    int64_t pool_pages, void* stream) {
  if (n < 0 || pool_pages < 0 || freq_rows < 0) return RM_ERR_SHAPE;
  if (n == 0) return RM_OK;
  if (!x || !weight || !dst_slot || !pool || (freqs && !position)) return RM_ERR_NULL;
  if (x_dtype != RM_F32 && x_dtype != RM_BF16) return RM_ERR_DTYPE;
  if (x_row_stride < kHeadDim && n > 1) return RM_ERR_SHAPE;
  const int esize = x_dtype == RM_BF16 ? 2 : 4;
  if (!aligned(x, 16) || ((x_row_stride * esize) & 15) || !aligned(pool, 16) ||
      (freqs && !aligned(freqs, 16)))
    return RM_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const int64_t rows = pool_pages * kPageRecords;
  if (x_dtype == RM_BF16)
    hipLaunchKernelGGL(native_store_kernel<true>, dim3(grid_for(n)), dim3(256), 0, s, x,
                       x_row_stride, weight, eps, dst_slot, position, freqs, freq_rows, n,
                       pool, rows);
  else
    hipLaunchKernelGGL(native_store_kernel<false>, dim3(grid_for(n)), dim3(256), 0, s, x,
                       x_row_stride, weight, eps, dst_slot, position, freqs, freq_rows, n,
                       pool, rows);
  return hipGetLastError() == hipSuccess ? RM_OK : RM_ERR_LAUNCH;
}
