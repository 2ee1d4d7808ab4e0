// Sparse-MLA decode over the paged latent pool: Direct (Packed 328-byte
// records, dequantized in the loader) and Native (584-byte records, control).
//
// Semantics (reference: FlashMLA sparse decode with the Remnant loader,
// third_party/README.md:260, 351-361; attention math training/losses.py:393-398,
// sink softmax test_integration.py:1620-1635): for query token t and head h,
//   K_j = reconstructed 512-d row of logical record indices[t, j] (V = K),
//   l_j = (q_h . K_j) * scale, Z = sum_j exp(l_j) + exp(sink_h),
//   out = sum_j exp(l_j) K_j / Z, lse = ln Z.
//
// Work split. A workgroup of six waves (eight for Packed splits at 16 heads)
// owns (split, token, 16-head block) and walks its share of the top-k list in
// stages of 32 records:
//   * record metadata (index -> block table -> page/row, validity) for the
//     share is resolved once into LDS; invalid records and slots past the end
//     point at a readable stand-in and are masked to zero;
//   * four producer waves each own 8 records of every stage. They copy the
//     record rows HBM -> LDS with global_load_lds three stages ahead (Packed
//     with a RoPE table: each lane also copies the 32 bytes of table row it
//     rotates with, two stages ahead, in the same in-order load stream) -- a
//     fixed number of loads per stage, so their waits are compile-time vmcnt
//     values -- and expand them into dense BF16 K rows in a four-slot LDS
//     ring: v_perm places the kept E4M3 codes (zeros for pruned coordinates)
//     from a 256-entry selector table, v_cvt_scalef32_pk_bf16_fp8 applies the
//     UE8M0 scale, the tail pairs are rotated (Packed: by the table row, or
//     with inverse frequencies by the cos and sin of the angle from the
//     record's position, computed in the lane) or copied as stored (Native);
//   * Packed splits at 16 heads add two tail waves: each expands and rotates
//     the 64-coordinate tails of 16 records of the stage straight from the
//     staged rows (in table mode with RoPE rows it loads into registers two
//     stages ahead), so the producers expand only the 448 other coordinates
//     and rotate nothing. By default they sit beside the two producers that
//     have no consumer beside them; on splits of several stages of at most
//     512 records beside the consumers, the producers paired on the other
//     two SIMDs (B=64 29.8 -> 27.9 us from positions, 29.9 -> 28.6 us from
//     the table);
//   * two consumer waves each own 256 of the 512 output coordinates. Both
//     compute S^T = K Q^T for every tile on v_mfma_f32_16x16x32_bf16 (Q in
//     registers), take weights against a fixed per-head reference (the first
//     valid stage's max) so O is never rescaled inside the loop, and
//     accumulate O += P K over the stage's 32 records on
//     v_mfma_f32_16x16x32_bf16 (K read with ds_read_b64_tr_b16). Weights up to
//     2^64 are far inside FP32/BF16 range; a split whose scores climb higher
//     is recomputed once against its true max;
//   * one workgroup barrier per stage hands the ring over: producers fill
//     stage s while consumers read stage s - 1. On splits of at most 512
//     records the producers run at a higher wave priority than the consumers
//     (with the default placement two SIMDs hold one of each, and the
//     producers set the stage time).
// A Packed record (328 B, 8-byte aligned) is fetched as the 21 aligned 16-byte
// pieces covering it: an even pool row from its start (its last piece reaches 8
// bytes into the next row of the same page, which always exists because row 63
// is odd), an odd row from 8 bytes before it, so it sits at staging offset 8.
// A Native record stages its 576-byte data row (36 pieces) and its scale row.
// A split count > 1 writes (O/l, m + log2 l) partials merged with the sink by a
// combine kernel; a single split finalises in place.
#include <mutex>
#include <type_traits>

#include "remnant_device.h"
#include "remnant_mi355x.h"

using namespace rm;

namespace {

constexpr int kT = 16;                     // records per tile
constexpr int kMaxSplits = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr uint64_t kAddrMask = (1ull << 58) - 1;
constexpr float kRefSlack = 64.0f;         // log2 headroom above the reference max

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

struct DecodeArgs {
  const uint16_t* q;
  const uint8_t* pool;     // contiguous pages, or the values plane [rows, 256]
  const uint8_t* bitmaps;  // planes: bitmaps [rows, 8] u64 and scales [rows, 8] u8
  const uint8_t* scales;
  int64_t pool_pages;      // pages of 64 records (planes: rows / 64, rounded up)
  int64_t pool_rows;
  const int32_t* block_table;
  int64_t bt_stride;
  int64_t max_blocks;
  const int32_t* seqlens;
  const int32_t* indices;
  int64_t topk;
  const int32_t* topk_length;
  const float* sink;
  const float* freqs;
  int64_t freq_rows;
  const float* inv_freq;   // position mode: [32] inverse frequencies (nullptr: identity)
  float scale_log2;
  int64_t q_len;
  int64_t heads;
  int chunk;       // records per split (multiple of 32)
  int splits;      // splits of this list (workgroups along x)
  int ws_splits;   // partial slots per row in the workspace; 0: finalise in place
  int ws_base;     // slot of this list's split 0
  uint16_t* out;
  float* lse;
  float* ws_o;     // [tokens, ws_splits, heads, 512]
  float* ws_lse;   // [tokens, ws_splits, heads]
};

// Two E4M3 codes (bytes 0-1, or 2-3 with kHi) times scale -> two BF16 (exact).
template <bool kHi>
__device__ __forceinline__ uint32_t cvt2(uint32_t codes, float scale) {
  return fp8_pair_to_bf16<kHi>(codes, scale);
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) const uint32_t lds_u32;

// Wait for every outstanding global load of this wave (LDS DMA included).
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0070); }
// LDS address (byte offset) of a shared-memory object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// 16 (or 4) bytes per lane, global -> LDS at lds + lane * size. The LDS address
// is passed as a plain number: the copies are tracked by the explicit waits in
// the tile loop (wait_vm_upto + barrier), and the compiler, not tying them to
// a particular array, adds no conservative waits of its own before LDS reads.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)(uintptr_t)__builtin_amdgcn_readfirstlane(lds),
                                   16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, uint32_t lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)(uintptr_t)__builtin_amdgcn_readfirstlane(lds),
                                   4, 0, 0);
}
// A 4-byte global -> LDS copy issued from inline assembly (M0 set and read in
// the same block, one wait state between). The compiler then sees no LDS DMA
// in flight in the issuing wave and adds no waits of its own before the
// wave's later LDS reads (before a ds_read_b64_tr_b16 it would otherwise wait
// for every outstanding copy); the wave waits for its copies explicitly. M0 is
// a reserved register the compiler may keep a value in across the block, so
// the block saves and restores it (the copy reads M0 when it issues).
__device__ __forceinline__ void dma4_opaque(const void* src, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds))
      : "memory");
}
// This lane's index from instructions the compiler cannot hoist: values
// derived from it are computed where they are used, not kept live across a
// loop whose registers are taken.
__device__ __forceinline__ int opaque_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Workgroup barrier for LDS data written by ordinary stores: this wave's LDS
// operations complete, then all waves meet. No memory-model fence: a release
// fence would also wait for every outstanding global load, including the
// copies of later tiles still in flight (their completion is ensured by the
// explicit wait_vm_upto before the tile barrier). The signal fences keep the
// compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void block_sync_lds() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited for
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Wait until at most N global loads of this wave are outstanding (loads
// complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vm_upto() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

constexpr int kPcProducers = 4;
constexpr int kPcMaxGroups = 2;            // 16-head groups per workgroup (1 or 2)
// Consumer waves and threads of a workgroup serving kHG groups of 16 heads:
// two consumer waves per group (one per half of the output coordinates), and
// with kHelp two tail waves (the Packed tails expanded and rotated apart from
// the expansion waves).
template <int kHG, bool kHelp = false>
struct PcRoles {
  static constexpr int kConsumers = 2 * kHG;
  static constexpr int kHelpers = kHelp ? 2 : 0;
  static constexpr int kThreads = 64 * (kConsumers + kPcProducers + kHelpers);
};
// Tail waves serve Packed splits at 16 heads (an eight-wave workgroup keeps
// 256 registers per wave).
template <bool kPacked, int kHG>
constexpr bool kTailWaves = kPacked && kHG == 1;
constexpr int kPcStage = 32;               // records per stage: two 16-record tiles
constexpr int kPcRing = 4;                 // K tile slots (two stages)
constexpr int kPcKPitch = kHeadDim + 16;   // BF16 per K row (1056 B: rows 8 banks apart)
// Within a K row, 8-coordinate chunk q sits at BF16 offset kchunk(q): even
// chunks in order from 0, odd chunks in order from kPcOddAt (4 banks past the
// matching even chunk). One pass of the expansion writes 32 even (or odd)
// chunks of a record contiguously, and the transposed reads of a 16-coordinate
// group (one even, one odd chunk, 4 rows) cover 32 distinct banks.
constexpr int kPcOddAt = 264;
__device__ __forceinline__ constexpr int kchunk(int q) { return (q >> 1) * 8 + (q & 1) * kPcOddAt; }
constexpr int kPcMaxChunk = 512;           // records per split
// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

template <bool kPacked>
struct PcGeo {
  static constexpr int kData = kPacked ? kRecordBytes : kNativeDataBytes;
  static constexpr int kPage = kPacked ? kPageBytes : kNativePageBytes;
  static constexpr int kPieces = kPacked ? 21 : kNativeDataBytes / 16;  // 16-B pieces per record
  static constexpr int kPitch = 16 * kPieces;                          // staged record pitch
  static constexpr int kRecPieces = 8 * kPieces;                       // one producer's 8 records
  static constexpr int kPieceCount = kRecPieces;
  static constexpr int kCopies = (kPieceCount + 63) / 64;              // 16-B copies per stage
  static constexpr int kScaleAt = 1024 * kCopies;                      // Native: scale rows
  static constexpr int kBuf = kScaleAt + (kPacked ? 0 : 256);          // bytes per stage buffer
  static constexpr int kDepth = 4;  // copy ring buffers (the step loop is unrolled by 4)
};

// Shared memory of one workgroup. The kernels declare one byte array of the
// larger format's size and view it as the format they run, so a kernel that
// runs either format per workgroup needs no more LDS than the larger one.
template <bool kPacked>
struct PcShared {
  using G = PcGeo<kPacked>;
  uint8_t raw[kPcProducers][G::kDepth][G::kBuf];  // copy ring (LDS address 0)
  uint16_t ktile[kPcRing][kT * kPcKPitch];
  // per record slot of the split, a ring of kPcMaxChunk entries (record i at
  // i % kPcMaxChunk; splits of more than kPcMaxChunk records refill it as they
  // go): pool row address, or (Q address | 1) for an invalid record or a slot
  // past the end (a readable stand-in source, odd so that bit 0 marks it);
  // Packed: RoPE row address (row 0 of the table for an invalid record, Q
  // without a table)
  uint64_t row_tab[kPcMaxChunk];
  uint64_t aux_tab[kPacked ? kPcMaxChunk : 1];
  // long splits: the records' top-k entries and block-table entries of the
  // next stages, copied in ahead of the table entries made from them
  int32_t idx_ring[3][64];
  int32_t bt_ring[3][64];
  uint64_t sel_tab[kPacked ? 256 : 1];
  // table mode in workgroups without tail waves (32 heads): per producer, a
  // two-stage ring of the RoPE row bytes its lanes rotate with ([stage %
  // 2][half][lane] 16 bytes); the tail waves hold their rows in registers
  alignas(16) uint8_t rope_ring[kPacked ? kPcProducers * 2 * 2 * 1024 : 1];
  float mrg[2 * kPcMaxGroups][2][16];  // consumers' (reference, seen) maxima per head
};
constexpr size_t kPcSmemBytes = sizeof(PcShared<true>) > sizeof(PcShared<false>)
                                    ? sizeof(PcShared<true>) : sizeof(PcShared<false>);

// Max of x over lanes col, col + 16, col + 32, col + 48 (col = lane % 16).
__device__ __forceinline__ float max_over_rows(float x) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = fmaxf(u2f(h[0]), u2f(h[1]));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(u2f(r[0]), u2f(r[1]));
}

// One workgroup's share: split `split` of list `a` (a C4 top-k list through
// the block table, or with a.block_table == nullptr a list of pool slots), for
// kHG groups of 16 heads: every expanded record serves all of them.
template <bool kPacked, int kHG, bool kPlanes = false, bool kLong = false, bool kPos = false,
          bool kHelp = false>
__device__ __forceinline__ void decode_pc(const DecodeArgs& a, PcShared<kPacked>* sm,
                                          const int split) {
  static_assert(!kHelp || kHG == 1, "tail waves: 16-head workgroups");
  static_assert(kPacked || !kPlanes, "planes hold Packed records");
  static_assert(kPacked || !kPos, "Native records store a rotated tail");
  using G = PcGeo<kPacked>;
  // global loads per stage in a producer's in-order stream: the copies, plus
  // the Native scale row or (table mode) the two Packed RoPE row loads
  // (table mode: the RoPE row loads, made by the tail waves when there are some)
  constexpr bool kRopeRows = kPacked && !kPos && !kHelp;
  constexpr int kRopeLoads = kRopeRows ? 2 : 0;
  constexpr int kLoads = G::kCopies + (kPacked ? kRopeLoads : 1);
  constexpr int kPcConsumers = PcRoles<kHG, kHelp>::kConsumers;
  constexpr int kPcThreads = PcRoles<kHG, kHelp>::kThreads;
  auto& ktile = sm->ktile;
  auto& raw = sm->raw;
  auto& sel_tab = sm->sel_tab;
  auto& row_tab = sm->row_tab;
  auto& aux_tab = sm->aux_tab;
  auto& mrg = sm->mrg;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Role index of this wave. A workgroup's waves fill SIMDs 0..3 in order
  // (hardware wave w on SIMD w % 4). By default the consumers are waves 0 and
  // 1, producers 0..3 waves 2..5 (2 and 3 beside the consumers) and tail
  // waves 6 and 7 (beside producers 0 and 1). Native workgroups of more than
  // one stage put the consumers on waves 2 and 3 (a SIMD each) and the
  // producers two per SIMD: the Native expansion is light enough to share a
  // SIMD with another one (B=64 33.6 -> 31.4 us, B=128 x next-n 2 119.9 ->
  // 109.1 us), the Packed one with its tail was not (35.5 -> 36.4), and
  // single-stage splits gain nothing from it. Decided from the launch
  // arguments alone, so the consumers' Q loads start at once.
  //
  // Packed workgroups with tail waves (eight waves) on splits of several
  // stages of at most 512 records: the tail waves take hardware waves 4 and 5
  // (beside the consumers on SIMDs 0 and 1) and producers 2 and 3 waves 6 and
  // 7 (two producers on each of SIMDs 2 and 3). A consumer slows less beside
  // a tail wave than beside a producer: B=64 29.7 -> 28.8 us (table) and 28.4
  // -> 28.0 us (positions). Long splits (B=128 x next-n 2 94 -> 98-102 us)
  // and single-stage splits (B=1) keep the default placement.
  const int wv_hw = uniform(tid >> 6);
  const bool several = (a.topk + kPcStage - 1) / kPcStage > (int64_t)a.splits;
  const bool remap = !kPacked && kHG == 1 && several;
  const bool tail_remap = kHelp && kPacked && !kLong && several;
  const int wv = remap ? (wv_hw == 2 ? 0 : wv_hw == 3 ? 1 : wv_hw < 2 ? wv_hw + 2 : wv_hw)
                 : tail_remap && wv_hw >= 4 ? (wv_hw ^ 2)
                                            : wv_hw;
  const int64_t t = blockIdx.y;
  const int64_t head_wg = (int64_t)blockIdx.z * 16 * kHG;
  // a consumer's 16 heads (consumers 2 hg and 2 hg + 1 serve group hg)
  const int64_t head0 = head_wg + (wv < kPcConsumers ? 16 * (wv >> 1) : 0);
  const int64_t b = t / a.q_len;

  int64_t len = a.topk;
  if (a.topk_length) {
    const int64_t l = a.topk_length[t];
    len = l < 0 ? 0 : (l < a.topk ? l : a.topk);
  }
  // this token's valid entries in whole stages, spread evenly over the splits
  // (at most a.chunk each, since len <= topk): a short list finishes early in
  // every split instead of emptying the last ones
  const int64_t len_stages = (len + kPcStage - 1) / kPcStage;
  const int64_t chunk = ((len_stages + a.splits - 1) / a.splits) * kPcStage;
  const int64_t k0 = (int64_t)split * chunk;
  const int64_t k1 = k0 + chunk < len ? k0 + chunk : len;
  const int n = k1 > k0 ? (int)(k1 - k0) : 0;
  const int stages = (n + kPcStage - 1) / kPcStage;
  const int64_t seqlen = a.seqlens ? a.seqlens[b] : INT64_MAX;

  // Consumers hold Q of the 16 heads as the B operand of S^T = K Q^T:
  // qf[ks] = Q[head lane % 16][32 ks + 8 (lane / 16) .. +7]
  bf16x8 qf[16];
  if (wv < kPcConsumers) {
    const uint16_t* qh = a.q + (t * a.heads + head0 + (lane & 15)) * kHeadDim + 8 * (lane >> 4);
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) qf[ks] = __builtin_bit_cast(bf16x8, *(const u32x4*)(qh + 32 * ks));
  }

  // ---- setup: selectors, record metadata ----
  if (kPacked && tid < 256) {
    const uint32_t e = tid;
    uint32_t r = 0;
    uint64_t sel = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool kept = (e >> (7 - i)) & 1u;
      sel |= (uint64_t)(kept ? r : 0x0cu) << (8 * i);
      r += kept ? 1u : 0u;
    }
    sel_tab[e] = sel;
  }
  const uint64_t stand_in = (uint64_t)a.q | 1u;
  const bool paged = a.block_table != nullptr;
  // whether logical record r of request b has a block-table entry to read
  auto in_table = [&](int64_t r) { return r >= 0 && r < seqlen && (r >> 6) < a.max_blocks; };
  // table entry of record slot i from its top-k entry r (< 0: none) and, for
  // a paged pool, its block-table entry pv (meaningful only when in_table(r))
  auto put_entry = [&](int i, int64_t r, int64_t pv) {
    bool ok;
    int64_t page;
    if (paged) {  // logical record of request b
      ok = in_table(r);
      page = ok ? pv : -1;
    } else {  // pool slot
      ok = r >= 0;
      page = r >> 6;
    }
    ok = ok && page >= 0 && page < a.pool_pages && page * 64 + (r & 63) < a.pool_rows;
    if (kPacked && a.freqs) ok = ok && r * 4 < a.freq_rows;
    // planes: the record's values row (16-byte aligned); its bitmap and scale
    // rows sit at a quarter and a 32nd of the values offset in their planes
    const uint8_t* pg = kPlanes ? a.pool + (ok ? page : 0) * 64 * kCodeBytes
                                : a.pool + (ok ? page : 0) * G::kPage;
    const int slot = i & (kPcMaxChunk - 1);
    row_tab[slot] = ok ? (uint64_t)(pg + (r & 63) * (kPlanes ? kCodeBytes : G::kData)) |
                             (kPacked ? 0 : (uint64_t)(r & 63) << 58)
                       : stand_in;
    // table mode: the record's RoPE row (row 0 of the table for an invalid
    // record, Q without a table); position mode: the position 4 r as a float
    // (0 for an invalid record, whose tail is zero)
    if (kPacked && kPos) aux_tab[slot] = f2u(ok ? (float)(4 * r) : 0.0f);
    else if (kPacked) aux_tab[slot] = a.freqs ? (uint64_t)(a.freqs + (ok ? r : 0) * 4 * 64) : (uint64_t)a.q;
  };
  // the first kPcMaxChunk slots, read directly by all threads
  constexpr int kEntries = (kPcMaxChunk + kPcThreads - 1) / kPcThreads;  // per thread
  auto build_table = [&]() {
    int64_t r[kEntries], pv[kEntries];
#pragma unroll
    for (int j = 0; j < kEntries; ++j) {  // top-k entries
      const int i = tid + j * kPcThreads;
      r[j] = -1;
      pv[j] = 0;
      if (i < kPcMaxChunk && i < n) r[j] = a.indices[t * a.topk + k0 + i];
    }
    // then every block-table entry, by unconditional loads (Q's first word
    // stands in where there is none): the compiler waits for a load made inside
    // a branch before the next one, which would serialise a thread's entries
#pragma unroll
    for (int j = 0; j < kEntries; ++j) {
      const bool has = paged && in_table(r[j]);
      const int32_t* src = has ? a.block_table + (b * a.bt_stride + (r[j] >> 6)) : (const int32_t*)a.q;
      const int32_t v = *src;
      pv[j] = has ? v : 0;
    }
#pragma unroll
    for (int j = 0; j < kEntries; ++j)
      if (tid + j * kPcThreads < kPcMaxChunk) put_entry(tid + j * kPcThreads, r[j], pv[j]);
  };
  // position mode: theta of the four RoPE pairs a producer lane rotates
  // (lane / 8 = j: pairs 4 j .. 4 j + 3; zero, the identity, without inverse
  // frequencies), loaded with the table and retired before the stage loop (the
  // empty asm reads it once, so the compiler's own wait for it is not repeated
  // inside the loop)
  // (tail waves: lane q = lane % 4 rotates the pairs 8 q .. 8 q + 7 of tail
  // chunks 2 q and 2 q + 1, theta and theta2)
  const bool tail_wave = kHelp && wv >= kPcConsumers + kPcProducers;
  f32x4 theta = {0.f, 0.f, 0.f, 0.f}, theta2 = theta;
  if (kPos && a.inv_freq) {
    if (tail_wave) {
      theta = *(const f32x4*)(a.inv_freq + 8 * (lane & 3));
      theta2 = *(const f32x4*)(a.inv_freq + 8 * (lane & 3) + 4);
    } else {
      theta = *(const f32x4*)(a.inv_freq + 4 * (lane >> 3));
    }
  }
  build_table();
  wait_vm();
  __syncthreads();
  if constexpr (kPos) asm volatile("" : "+v"(theta), "+v"(theta2));

  // Splits of more than kPcMaxChunk records: consumer 0 refills the table
  // ring ahead of the producers, after its MFMA work of each step s. It
  // copies the top-k entries of stage s + 6 into LDS, copies the block-table
  // entries of stage s + 5 (from the top-k entries copied a step earlier), and
  // writes the table entries of stage s + 4, whose copies the producers issue
  // at step s + 1, after the barrier. Slot i % kPcMaxChunk then belongs to
  // stage i / kPcStage - 16, consumed at step s - 11. The copies go through
  // inline assembly with this wave's own waits, so the compiler adds none
  // before the MFMA loop's transposed LDS reads.
  constexpr int kRingStages = kPcMaxChunk / kPcStage;
  const bool long_split = kLong && stages > kRingStages;
  auto refill = [&](int s) {
    wait_vm();  // this wave's copies of the previous step have landed
    const int ln = opaque_lane();
    int q = s + 4;
    if (q >= kRingStages && q < stages && ln < kPcStage) {
      const int i = q * kPcStage + ln;
      const int64_t r = i < n ? (int64_t)sm->idx_ring[q % 3][ln] : -1;
      put_entry(i, r, sm->bt_ring[q % 3][ln]);
    }
    q = s + 5;
    if (q >= kRingStages && q < stages) {
      const int i = q * kPcStage + ln;
      const int64_t r = ln < kPcStage && i < n ? (int64_t)sm->idx_ring[q % 3][ln] : -1;
      const int32_t* src = paged && in_table(r) ? a.block_table + (b * a.bt_stride + (r >> 6))
                                                : (const int32_t*)a.q;
      dma4_opaque(src, lds_addr(&sm->bt_ring[q % 3][0]));
    }
    q = s + 6;
    if (q >= kRingStages && q < stages) {
      const int i = q * kPcStage + ln;
      const int32_t* src = ln < kPcStage && i < n ? a.indices + (t * a.topk + k0 + i)
                                                  : (const int32_t*)a.q;
      dma4_opaque(src, lds_addr(&sm->idx_ring[q % 3][0]));
    }
  };

  // Overflow test on the consumers' published (reference, seen) maxima: a
  // workgroup-uniform decision every wave takes from LDS.
  auto redo_pass = [&](float& mtrue) {
    const int h = lane & 15;
    bool over = false;
#pragma unroll
    for (int c = 0; c < kPcConsumers; ++c) over = over || mrg[c][1][h] > mrg[c][0][h] + kRefSlack;
    const int c0 = wv < kPcConsumers ? wv & ~1 : 0;  // this consumer's group
    mtrue = fmaxf(mrg[c0][1][h], mrg[c0 + 1][1][h]);
    return __ballot(over) != 0;
  };

  // The roles run separate loops with the same barrier sequence per pass
  // (stages + 1 ring barriers, then two around the overflow test), so consumer
  // state (O) is never live in producers.
  if constexpr (kHelp && !kPacked) {
    if (tail_wave) {
      // A launch with tail waves that runs a Native split here (the window
      // rows of a joint launch): they only keep the barrier sequence.
      for (int pass = 0; pass < 2; ++pass) {
        for (int s = 0; s <= stages; ++s) block_sync_lds();
        if (stages <= 1) break;
        __syncthreads();
        float mtrue;
        const bool redo = redo_pass(mtrue);
        __syncthreads();
        if (!redo) break;
        if (long_split) {
          build_table();
          wait_vm();
          __syncthreads();
        }
      }
      return;
    }
  }
  if constexpr (kHelp && kPacked) {
    if (tail_wave) {
      // ================= tail wave =================
      // Tail wave hh expands and rotates the 64-coordinate tails (bitmap word
      // 7) of the 16 records of expansion waves 2 hh and 2 hh + 1, straight
      // from their staged rows: lane (record k = lane / 4, quarter q = lane %
      // 4) does tail chunks 2 q and 2 q + 1 (RoPE pairs 8 q .. 8 q + 7). The
      // stage's copies have landed once its ring barrier is passed (every
      // expansion wave waits for its own before the barrier), and the
      // expansion waves write no tail chunk, so the step needs no other
      // synchronisation. Beside the producers (the default placement) the
      // tail waves issue ahead of them (B=64 29.1 -> 28.8 us from positions
      // before the placement above, B=128 x next-n 2 94.7 -> 92.5 us from the
      // table); beside the consumers they keep the default priority.
      if (!tail_remap) __builtin_amdgcn_s_setprio(3);
      const int hh = wv - kPcConsumers - kPcProducers;
      const int k = lane >> 2, q = lane & 3;
      const int pp = 2 * hh + (k >> 3), pi = k & 7;
      // Table mode: the lane loads bytes 64 q .. 64 q + 63 of its record's
      // RoPE row into registers, two stages ahead (two register sets, even
      // and odd stages; stages past the end load Q). The tail waves issue no
      // LDS copies, so the compiler's own waits for these loads are exact.
      using Rows = f32x4[4];
      auto tload = [&](int s, Rows& r) {
        const int slot = (s * kPcStage + 8 * pp + pi) & (kPcMaxChunk - 1);
        const uint64_t row = s < stages ? aux_tab[slot] : (uint64_t)a.q;
#pragma unroll
        for (int u = 0; u < 4; ++u)  // global (not flat) loads: counted by vmcnt alone
          r[u] = *(const __attribute__((address_space(1))) f32x4*)(row + 64 * q + 16 * u);
      };
      auto tail = [&](int s, auto bufc, const Rows& rr) {
        constexpr int B = decltype(bufc)::value;
        const uint8_t* st = &raw[pp][B][0] + pi * G::kPitch;
        const int slot = (s * kPcStage + 8 * pp + pi) & (kPcMaxChunk - 1);
        const uint64_t row = row_tab[slot];
        const bool valid = !(row & 1u), odd = !kPlanes && (row & 8u) != 0;
        const bool sodd = kPlanes ? (((row - (uint64_t)a.pool) >> 8) & 1u) != 0 : odd;
        // codes and bitmap of a contiguous record from an odd pool row sit 8
        // bytes in; planes stage the bitmap at 256 and the scale row at 320
        const uint8_t* bm = st + kCodeBytes + (odd ? 8 : 0);
        const uint64_t wa = *(const uint64_t*)(bm + 16 * q);
        const uint64_t wb = *(const uint64_t*)(bm + 16 * q + 8);
        const uint64_t w7r = *(const uint64_t*)(bm + 56);
        const uint32_t sw = *(const uint32_t*)(st + kDataBytes + (sodd ? 8 : 0) + 4);
        const uint64_t w7 = valid ? w7r : 0u;
        // codes before the tail: the record's total (its four lanes' words)
        // less word 7's
        int cnt = valid ? __popcll(wa) + __popcll(wb) : 0;
        cnt += __builtin_amdgcn_update_dpp(0, cnt, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
        cnt += __builtin_amdgcn_update_dpp(0, cnt, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
        const int before = cnt - __popcll(w7);
        // chunk c of word 7 is byte 7 - c (coordinate i of it: bit 7 - i)
        const uint32_t b0 = (uint32_t)(w7 >> (56 - 16 * q)) & 0xffu;
        const uint32_t b1 = (uint32_t)(w7 >> (48 - 16 * q)) & 0xffu;
        const int pre0 = q == 0 ? 0 : __popcll((w7 >> 1) >> (63 - 16 * q));  // bytes 7 .. 8 - 2q
        const float scale = exp2i((int)(valid ? sw >> 24 : 0u) - 127);
        uint16_t* const krow = &ktile[(2 * s + (pp >> 1)) % kPcRing][0] +
                               (8 * (pp & 1) + pi) * kPcKPitch;
        const uint32_t r0 = lds_addr(st) + (odd ? 8u : 0u) + (uint32_t)(before + pre0);
        const uint32_t r1 = r0 + (uint32_t)__popc(b0);
        // (cos, sin) of the eight pairs: from the position (0 for an invalid
        // record, whose tail is zero), or from the table row (the identity
        // without a table)
        float cs[16];
        if constexpr (kPos) {
          const float pos = u2f((uint32_t)aux_tab[slot]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            rope_sincos(pos * theta[e], cs[2 * e + 1], cs[2 * e]);
            rope_sincos(pos * theta2[e], cs[8 + 2 * e + 1], cs[8 + 2 * e]);
          }
        } else {
          const bool rope = a.freqs != nullptr;
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) cs[4 * u + e] = rope ? rr[u][e] : ((e & 1) ? 0.f : 1.f);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t r = h ? r1 : r0;
          const lds_u32* cw = (const lds_u32*)(uintptr_t)(r & ~3u);
          const uint64_t sel = sel_tab[h ? b1 : b0];
          const uint32_t lo4 = __builtin_amdgcn_alignbyte(cw[1], cw[0], r);
          const uint32_t hi4 = __builtin_amdgcn_alignbyte(cw[2], cw[1], r);
          const uint32_t lo = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)sel);
          const uint32_t hi = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)(sel >> 32));
          const u32x4 v = {cvt2<false>(lo, scale), cvt2<true>(lo, scale), cvt2<false>(hi, scale),
                           cvt2<true>(hi, scale)};
          float x8[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x8[2 * e] = u2f(v[e] << 16);
            x8[2 * e + 1] = u2f(v[e] & 0xffff0000u);
          }
          rope4(x8, cs + 8 * h);
          const bf16x8 rot = {(__bf16)x8[0], (__bf16)x8[1], (__bf16)x8[2], (__bf16)x8[3],
                              (__bf16)x8[4], (__bf16)x8[5], (__bf16)x8[6], (__bf16)x8[7]};
          *(bf16x8*)(krow + kchunk(kNopeDim / 8 + 2 * q + h)) = rot;
        }
      };
      // step s: the tail of stage s from its rows, then the rows of s + 2 into
      // the same registers
      auto tstep = [&](int s, auto bufc, Rows& rr) {
        block_sync_lds();  // the stage's copies landed, its ring slots free
        if (s < stages) tail(s, bufc, rr);
        if constexpr (!kPos) tload(s + 2, rr);
      };
      for (int pass = 0; pass < 2; ++pass) {
        Rows ra, rb;  // rows of the even and odd stages (table mode)
        if constexpr (!kPos) {
          tload(0, ra);
          tload(1, rb);
        }
        for (int s0 = 0; s0 <= stages; s0 += 4) {
          tstep(s0, std::integral_constant<int, 0>{}, ra);
          if (s0 + 1 <= stages) tstep(s0 + 1, std::integral_constant<int, 1>{}, rb);
          if (s0 + 2 <= stages) tstep(s0 + 2, std::integral_constant<int, 2>{}, ra);
          if (s0 + 3 <= stages) tstep(s0 + 3, std::integral_constant<int, 3>{}, rb);
        }
        wait_vm();  // the loads past the end
        if (stages <= 1) break;  // as the other roles
        __syncthreads();  // consumers' maxima published
        float mtrue;
        const bool redo = redo_pass(mtrue);
        __syncthreads();
        if (!redo) break;
        if (long_split) {
          build_table();
          wait_vm();
          __syncthreads();
        }
      }
      return;
    }
  }
  if (wv >= kPcConsumers) {
    // ================= producer =================
    constexpr int D = G::kDepth;
    static_assert(D == 4, "the stage loop below is unrolled for a four-buffer ring");
    const int p = wv - kPcConsumers;
    // Producers issue ahead of the consumers on the SIMDs they share (two of
    // them hold a consumer and a producer each): the arbiter otherwise favours
    // the older consumer waves, while the producers' expansion sets the stage
    // time (interleaved runs: Packed B=64 33.2-33.8 -> 31.3-32.2 us, the
    // reference H64/H128 shapes 0.2-1.5 us faster, Native and B=1 unchanged).
    // Long splits keep equal priorities: their consumer wave 0 also refills
    // the record table, and with the producers ahead B=128 x next-n 2 ran 8 %
    // slower.
    if constexpr (!kLong) __builtin_amdgcn_s_setprio(2);
    const uint8_t* const dummy = (const uint8_t*)a.q;
    // Copies of stage s into ring buffer B: the record table entries first,
    // then a fixed number of copies per stage. Invalid records and slots past
    // the end copy from the stand-in (Q); the expansion masks them.
    auto issue_stage = [&](int s, auto bufc) {
      constexpr int B = decltype(bufc)::value;
      const uint32_t base = lds_addr(&raw[p][B][0]);
      const int rec0 = s * kPcStage + 8 * p;
      uint64_t rw[G::kCopies];
#pragma unroll
      for (int j = 0; j < G::kCopies; ++j) {
        const int c = lane + 64 * j;
        const int r = c < G::kRecPieces ? c / G::kPieces : 0;
        const int idx = (rec0 + r) & (kPcMaxChunk - 1);
        rw[j] = c >= G::kPieceCount ? (uint64_t)a.q : row_tab[idx];
      }
      uint64_t srow = 0;
      if (!kPacked) srow = row_tab[(rec0 + ((lane >> 1) & 7)) & (kPcMaxChunk - 1)];
#pragma unroll
      for (int j = 0; j < G::kCopies; ++j) {
        const int c = lane + 64 * j;
        uint64_t src;
        if (c < G::kRecPieces) {
          const int piece = c - (c / G::kPieces) * G::kPieces;
          if (kPlanes && !(rw[j] & 1u)) {  // codes 0..15, bitmap 16..19, scales 20
            const uint64_t off = rw[j] - (uint64_t)a.pool;  // slot * 256
            src = piece < 16 ? rw[j] + 16 * piece
                  : piece < 20 ? (uint64_t)a.bitmaps + (off >> 2) + 16 * (piece - 16)
                               : (uint64_t)a.scales + ((off >> 5) & ~(uint64_t)15);
          } else {
            src = (rw[j] & (kPacked ? ~(uint64_t)15 : kAddrMask & ~(uint64_t)15)) + 16 * piece;
          }
        } else {  // a filler lane
          src = rw[j];
        }
        dma16((const void*)src, base + 1024 * j);
      }
      if (!kPacked) {
        const uint32_t rip = (uint32_t)(srow >> 58);
        const bool ok = lane < 16 && !(srow & 1u);
        const uint8_t* src = ok ? (const uint8_t*)(srow & kAddrMask) - rip * G::kData +
                                      kPageRecords * G::kData + rip * kScaleBytes + 4 * (lane & 1)
                                : dummy;
        dma4(src, base + G::kScaleAt);
      }
    };

    // ---- Packed expansion ----
    // Lane (record i = lane % 8, word w = lane / 8) expands the 64 coordinates
    // of bitmap word w of record i: first reads (head), code windows and
    // selectors (gather), conversion into the K ring (expand), tail rotation.
    struct Head {  // first reads: record slot, bitmap word and scales at both offsets
      uint64_t row;
      uint32_t w[4], sc0, sc1;
    };
    struct Gath {  // code windows and selectors of the 8 chunks of this lane's word
      uint32_t d0[8], d1[8], d2[8], rk[8];
      uint64_t sel[8];
      float scale;
    };
    const int pi = lane & 7, pw = lane >> 3;
    auto head = [&](int s, auto bufc, Head& h) {
      constexpr int B = decltype(bufc)::value;
      const uint8_t* st = &raw[p][B][0] + pi * G::kPitch;
      h.row = row_tab[(s * kPcStage + 8 * p + pi) & (kPcMaxChunk - 1)];
      // a record staged from an odd pool row starts 8 bytes in
#pragma unroll
      for (int e = 0; e < 4; ++e) h.w[e] = *(const uint32_t*)(st + kCodeBytes + 8 * pw + 4 * e);
      h.sc0 = *(const uint32_t*)(st + kDataBytes + 4 * (pw >> 2));
      h.sc1 = *(const uint32_t*)(st + kDataBytes + 8 + 4 * (pw >> 2));
    };
    auto gather = [&](auto bufc, const Head& h, Gath& gt) {
      constexpr int B = decltype(bufc)::value;
      const uint8_t* st = &raw[p][B][0] + pi * G::kPitch;
      // odd: codes and bitmap staged 8 bytes in (a contiguous record from an
      // odd pool row); sodd: the scales 8 bytes in (planes: an odd slot)
      const bool valid = !(h.row & 1u), odd = !kPlanes && (h.row & 8u) != 0;
      const bool sodd = kPlanes ? (((h.row - (uint64_t)a.pool) >> 8) & 1u) != 0 : odd;
      const uint32_t wlo = valid ? (odd ? h.w[2] : h.w[0]) : 0u;
      const uint32_t whi = valid ? (odd ? h.w[3] : h.w[1]) : 0u;
      const uint32_t sw = valid ? (sodd ? h.sc1 : h.sc0) : 0u;
      gt.scale = exp2i((int)((sw >> (8 * (pw & 3))) & 0xffu) - 127);
      // codes before this word: exclusive prefix over the record's lanes
      // i + 8 w. A 16-lane row holds words 2k, 2k + 1: pair sums in the row
      // (DPP), row totals combined across rows with the permlane swaps.
      const int cnt = __popc(wlo) + __popc(whi);
      const int y = cnt + __builtin_amdgcn_update_dpp(0, cnt, 0x118, 0xf, 0xf, true);  // row_shr:8
      const int t8 = __builtin_amdgcn_update_dpp(0, y, 0x108, 0xf, 0xf, true);         // row_shl:8
      const int tot = (pw & 1) ? y : t8;  // words 2k + 2k+1, in every lane of row k
      const auto hs = __builtin_amdgcn_permlane16_swap((uint32_t)tot, (uint32_t)tot, false, false);
      const int other = (pw & 2) ? (int)hs[0] : (int)hs[1];  // total of the paired row
      int before = (pw & 2) ? other : 0;
      const int pair = tot + other;  // rows 0+1 or 2+3
      const auto qs = __builtin_amdgcn_permlane32_swap((uint32_t)pair, (uint32_t)pair, false, false);
      before += (pw & 4) ? (int)qs[0] : 0;
      // LDS byte address of the next code: the staged record (4-byte aligned)
      // plus the codes before it; its low two bits align the code window
      uint32_t r = lds_addr(st) + (odd ? 8u : 0u) + (uint32_t)(before + y - cnt);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t byte = c < 4 ? (whi >> (24 - 8 * c)) & 0xffu : (wlo >> (56 - 8 * c)) & 0xffu;
        const lds_u32* cw = (const lds_u32*)(uintptr_t)(r & ~3u);
        gt.d0[c] = cw[0];
        gt.d1[c] = cw[1];
        gt.d2[c] = cw[2];
        gt.sel[c] = sel_tab[byte];
        gt.rk[c] = r;
        r += __popc(byte);
      }
    };
    auto expand = [&](int s, const Gath& gt) {
      uint16_t* const krow =
          &ktile[(2 * s + (p >> 1)) % kPcRing][0] + (8 * (p & 1) + pi) * kPcKPitch;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t lo4 = __builtin_amdgcn_alignbyte(gt.d1[c], gt.d0[c], gt.rk[c]);
        const uint32_t hi4 = __builtin_amdgcn_alignbyte(gt.d2[c], gt.d1[c], gt.rk[c]);
        const uint32_t lo = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)gt.sel[c]);
        const uint32_t hi = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)(gt.sel[c] >> 32));
        // (with tail waves, word 7 -- the tail -- is theirs)
        if (!kHelp || pw != 7)
          *(u32x4*)(krow + kchunk(8 * pw + c)) =
              u32x4{cvt2<false>(lo, gt.scale), cvt2<true>(lo, gt.scale), cvt2<false>(hi, gt.scale),
                    cvt2<true>(hi, gt.scale)};
      }
    };
    // Table mode: lane (i, j) copies bytes 32 j .. 32 j + 31 of record i's
    // RoPE row (the (cos, sin) of pairs 4j..4j+3) HBM -> LDS into its own two
    // 16-byte slots of a two-stage ring, two stages ahead, after the stage's
    // copies. For stages past the end it copies from Q (the loads per stage
    // stay fixed). Slot S is refilled at the step that rotated from it, after
    // that rotation's reads returned. Position mode loads nothing: the lane
    // holds theta of its four pairs and computes the angles.
    auto rope_slot = [&](int S) { return &sm->rope_ring[(p * 2 + S) * 2 * 1024 + 16 * lane]; };
    auto issue_rope = [&](int s, auto slotc) {
      constexpr int S = decltype(slotc)::value;
      const uint64_t entry = aux_tab[(s * kPcStage + 8 * p + pi) & (kPcMaxChunk - 1)];
      const uint64_t row = s < stages ? entry : (uint64_t)a.q;
      const uint32_t base = lds_addr(&sm->rope_ring[(p * 2 + S) * 2 * 1024]);
      dma16((const void*)(row + 32 * pw), base);
      dma16((const void*)(row + 32 * pw + 16), base + 1024);
    };
    // loads issued after the RoPE copies of stage s when stage s is rotated: the
    // copies of stage s + 2, the RoPE copies of stage s + 1, the copies of s + 3
    constexpr int kRopeLag = 2 * G::kCopies + 2;
    auto rope_ready = [&]() {
      wait_vm_upto<kRopeLag>();
      wave_lds_sync();
    };
    // tail: lane (i, j) rotates pairs 4j..4j+3 of record i (BF16 in, BF16 out);
    // an invalid record's tail is zero and its stand-in RoPE row finite; without
    // a table the rotation is the identity
    auto rotate = [&](int s, auto bufc) {
      constexpr int B = decltype(bufc)::value;
      wave_lds_sync();
      uint16_t* const tail = &ktile[(2 * s + (p >> 1)) % kPcRing][0] +
                             (8 * (p & 1) + pi) * kPcKPitch + kchunk(kNopeDim / 8 + pw);
      const u32x4 v = *(const u32x4*)tail;
      float cs[8];
      if constexpr (kPos) {  // angle RN(4 r * theta_j) of pairs 4 pw .. 4 pw + 3
        const float pos = u2f((uint32_t)aux_tab[(s * kPcStage + 8 * p + pi) & (kPcMaxChunk - 1)]);
#pragma unroll
        for (int e = 0; e < 4; ++e) rope_sincos(pos * theta[e], cs[2 * e + 1], cs[2 * e]);
      } else {
        rope_ready();
        const uint8_t* slot = rope_slot(B & 1);
        const f32x4 f0 = *(const f32x4*)slot;
        const f32x4 f1 = *(const f32x4*)(slot + 1024);
        const bool rope = a.freqs != nullptr;
        const float t[8] = {rope ? f0[0] : 1.f, rope ? f0[1] : 0.f, rope ? f0[2] : 1.f,
                            rope ? f0[3] : 0.f, rope ? f1[0] : 1.f, rope ? f1[1] : 0.f,
                            rope ? f1[2] : 1.f, rope ? f1[3] : 0.f};
#pragma unroll
        for (int e = 0; e < 8; ++e) cs[e] = t[e];
      }
      float x8[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x8[2 * e] = u2f(v[e] << 16);
        x8[2 * e + 1] = u2f(v[e] & 0xffff0000u);
      }
      rope4(x8, cs);
      const bf16x8 rot = {(__bf16)x8[0], (__bf16)x8[1], (__bf16)x8[2], (__bf16)x8[3],
                          (__bf16)x8[4], (__bf16)x8[5], (__bf16)x8[6], (__bf16)x8[7]};
      *(bf16x8*)tail = rot;
    };

    // ---- Native expansion: stored codes and rotated tail, per stage ----
    auto produce_native = [&](int s, auto bufc) {
      constexpr int B = decltype(bufc)::value;
        // lane (record i, word w) converts the 64 coordinates of word w; piece
        // pairs in the order (c + w / 2) % 4 keep a record's lanes on distinct banks
        const int ni = lane >> 3, nw = lane & 7;
        const bool nvalid = !(row_tab[(s * kPcStage + 8 * p + ni) & (kPcMaxChunk - 1)] & 1u);
        const uint8_t* const rb = &raw[p][B][0];
        const uint8_t* nst = rb + ni * G::kPitch;
        uint16_t* const nrow =
            &ktile[(2 * s + (p >> 1)) % kPcRing][0] + (8 * (p & 1) + ni) * kPcKPitch;
        const uint32_t sw0 = *(const uint32_t*)(rb + G::kScaleAt + 8 * ni + 4 * (nw >> 2));
        u32x4 in0[4], in1[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // Nope word: 16 codes per piece; tail: 8 BF16 x 2
          const int cc = (c + (nw >> 1)) & 3;
          const uint8_t* src = nw < 7 ? nst + 64 * nw + 16 * cc : nst + kNopeDim + 32 * cc;
          in0[c] = *(const u32x4*)src;
          in1[c] = *(const u32x4*)(src + 16);
        }
        const uint32_t sw = nvalid ? sw0 : 0u;
        const float scale = exp2i((int)((sw >> (8 * (nw & 3))) & 0xffu) - 127);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int cc = (c + (nw >> 1)) & 3;
          u32x4 out0, out1;
          if (nw < 7) {  // 16 E4M3 codes -> two 8-coordinate chunks
            const u32x4 codes = nvalid ? in0[c] : u32x4{0u, 0u, 0u, 0u};
            out0 = u32x4{cvt2<false>(codes[0], scale), cvt2<true>(codes[0], scale),
                         cvt2<false>(codes[1], scale), cvt2<true>(codes[1], scale)};
            out1 = u32x4{cvt2<false>(codes[2], scale), cvt2<true>(codes[2], scale),
                         cvt2<false>(codes[3], scale), cvt2<true>(codes[3], scale)};
          } else {  // tail: rotated BF16 as stored
            out0 = nvalid ? in0[c] : u32x4{0u, 0u, 0u, 0u};
            out1 = nvalid ? in1[c] : u32x4{0u, 0u, 0u, 0u};
          }
          *(u32x4*)(nrow + kchunk(8 * nw + 2 * cc)) = out0;
          *(u32x4*)(nrow + kchunk(8 * nw + 2 * cc + 1)) = out1;
        }
    };

    // Native workgroups with paired expansion waves: waves 2 and 3 (each the
    // second of a SIMD's pair) issue their copies after their stage's work,
    // so the pair's first LDS waits of a stage do not coincide (B=64 27.6 ->
    // 27.3 us, B=128 x next-n 2 93.3 -> 90.9 us). The Packed pairs, beside
    // the tail waves' copies and reads, ran 1-3 % slower with it.
    const bool late_copies = remap && p >= 2;
    // One stage step in ring phase B (the stage loop is unrolled by D so the
    // ring buffer of each step is fixed).
    auto step = [&](int s, auto bufc) {
      constexpr int B = decltype(bufc)::value;
      // this wave's copies of stage s are done once at most the loads issued
      // after them remain outstanding: the later D - 2 stages' loads (Packed:
      // and the RoPE loads of stage s - 1, issued right after the copies)
      wait_vm_upto<(D - 2) * kLoads + kRopeLoads>();
      wave_lds_sync();
      block_sync_lds();  // ring slots of stage s free (consumers are on stage s - 1)
      // past the end: fillers
      if (!late_copies)
        issue_stage(s + D - 1, std::integral_constant<int, (B + D - 1) % D>{});
      if (s < stages) {
        if constexpr (kPacked) {
          Head h;
          Gath gt;
          head(s, bufc, h);
          gather(bufc, h, gt);
          expand(s, gt);
          if constexpr (!kHelp) rotate(s, bufc);
        } else {
          produce_native(s, bufc);
        }
      }
      if (late_copies)
        issue_stage(s + D - 1, std::integral_constant<int, (B + D - 1) % D>{});
      if constexpr (kRopeRows) issue_rope(s + 2, std::integral_constant<int, B & 1>{});
    };

    for (int pass = 0; pass < 2; ++pass) {
      // the loads of steps -3 .. -1: copies of stages 0..2, each followed by
      // two RoPE loads (stage -1: two copies of Q into the idle ring buffer 3)
      issue_stage(0, std::integral_constant<int, 0>{});
      if constexpr (kRopeRows) {
        const uint32_t idle = lds_addr(&raw[p][D - 1][0]);
        dma16(a.q, idle);
        dma16(a.q, idle + 1024);
      }
      issue_stage(1, std::integral_constant<int, 1>{});
      if constexpr (kRopeRows) issue_rope(0, std::integral_constant<int, 0>{});
      issue_stage(2, std::integral_constant<int, 2>{});
      if constexpr (kRopeRows) issue_rope(1, std::integral_constant<int, 1>{});
      for (int s0 = 0; s0 <= stages; s0 += D) {
        step(s0, std::integral_constant<int, 0>{});
        if (s0 + 1 <= stages) step(s0 + 1, std::integral_constant<int, 1>{});
        if (s0 + 2 <= stages) step(s0 + 2, std::integral_constant<int, 2>{});
        if (s0 + 3 <= stages) step(s0 + 3, std::integral_constant<int, 3>{});
      }
      wait_vm();  // drain the filler copies (and the RoPE copies past the end)
      if (stages <= 1) break;  // as the consumers: no second pass
      __syncthreads();  // consumers' maxima published
      float mtrue;
      const bool redo = redo_pass(mtrue);
      __syncthreads();
      if (!redo) break;
      if (long_split) {  // the ring holds the last stages: rebuild the first ones
        build_table();
        wait_vm();
        __syncthreads();
      }
    }
    return;
  }

  // ================= consumer =================
  // Consumer c owns output coordinates 256 c .. 256 c + 255 of the 16 heads.
  // Both consumers score every tile, so their softmax state (reference, sum)
  // is identical and each finalises its half of O on its own.
  const int g = lane >> 4, col = lane & 15;
  const int half = wv & 1;  // 0 or 1
  f32x4 o[16];          // O[head 4g + i][256 half + 16 nt + col]
  float m_ref = -INFINITY, m_seen = -INFINITY, l_run = 0.0f;

  // One stage: tiles 2s' and 2s' + 1 of the ring (slots sa, sb; records
  // tile0 .. tile0 + 31). S^T for each tile on v_mfma_f32_16x16x32_bf16, then
  // O[:, half] += P K over the 32 records on v_mfma_f32_16x16x32_bf16: lane
  // (g, col) holds P[head col][records 4g .. 4g+3 of both tiles] -- exactly the
  // A operand with k = 8 g + j <-> (tile j / 4, record 4 g + j % 4) -- and the
  // B operand is the two transposed K reads of the same records. Branch-free,
  // so the scheduling groups at the end can pipeline the LDS reads.
  auto consume = [&](int sa, int sb, int tile0) {
    const uint16_t* kta = &ktile[sa][0];
    const uint16_t* ktb = &ktile[sb][0];
    const uint64_t ra = row_tab[(tile0 + col) & (kPcMaxChunk - 1)];
    const uint64_t rb = row_tab[(tile0 + kT + col) & (kPcMaxChunk - 1)];
    const uint64_t va = __ballot(lane < kT && !(ra & 1u));
    const uint64_t vb = __ballot(lane < kT && !(rb & 1u));
    const int ko = col * kPcKPitch + kchunk(g);  // chunk 4 ks + g at ko + 16 ks
    const uint16_t* kra = kta + ko;
    const uint16_t* krb = ktb + ko;
    f32x4 sa4 = {0.f, 0.f, 0.f, 0.f}, sb4 = sa4;  // lane: S^T[rec 4g + i][head col]
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {  // two independent accumulation chains
      sa4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, *(const u32x4*)(kra + 16 * ks)), qf[ks], sa4, 0, 0, 0);
      sb4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, *(const u32x4*)(krb + 16 * ks)), qf[ks], sb4, 0, 0, 0);
    }
    float sv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[i] = ((va >> (4 * g + i)) & 1u) ? sa4[i] * a.scale_log2 : -INFINITY;
      sv[4 + i] = ((vb >> (4 * g + i)) & 1u) ? sb4[i] * a.scale_log2 : -INFINITY;
    }
    float mt = sv[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mt = fmaxf(mt, sv[i]);
    m_seen = fmaxf(m_seen, mt);
    // reference: the first stage with a valid record sets it for every head
    mt = max_over_rows(mt);
    m_ref = m_ref == -INFINITY ? mt : m_ref;
    const float mr = m_ref == -INFINITY ? 0.0f : m_ref;
    float pr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pr[i] = __builtin_amdgcn_exp2f(sv[i] - mr);
      l_run += pr[i];
    }
    const bf16x8 pa = {(__bf16)pr[0], (__bf16)pr[1], (__bf16)pr[2], (__bf16)pr[3],
                       (__bf16)pr[4], (__bf16)pr[5], (__bf16)pr[6], (__bf16)pr[7]};
    // coordinates 256 half + 16 nt + 4 (col % 4) .. + 3 of record row 4g + col / 4:
    // chunk 32 half + 2 nt + (col % 4) / 2 at vo + 8 nt
    const int vo = (4 * g + (col >> 2)) * kPcKPitch + kchunk(((col & 3) >> 1) + 32 * half) +
                   4 * (col & 1);
#pragma unroll
    for (int nt = 0; nt < 16; ++nt) {
      const s16x4 ka = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(kta + vo + 8 * nt));
      const s16x4 kb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(ktb + vo + 8 * nt));
      const s16x8 kab = {ka[0], ka[1], ka[2], ka[3], kb[0], kb[1], kb[2], kb[3]};
      o[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, __builtin_bit_cast(bf16x8, kab), o[nt],
                                                      0, 0, 0);
    }
    // S: K reads run 8 ahead of the MFMAs; the first 8 PV reads overlap the
    // last S MFMAs and the softmax; PV reads then run 8 ahead.
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8, 0);
#pragma unroll
    for (int k = 0; k < 24; ++k) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8, 0);
#pragma unroll
    for (int k = 0; k < 12; ++k) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4, 0);
  };

  // Pass 0 takes the reference from the first valid stage; a split whose
  // scores exceed it by more than 2^kRefSlack is recomputed once against its
  // true max.
  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int nt = 0; nt < 16; ++nt) o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    l_run = 0.0f;
    for (int s = 0; s <= stages; ++s) {
      block_sync_lds();  // stage s - 1 in the ring
      if (s >= 1) consume((2 * s - 2) % kPcRing, (2 * s - 1) % kPcRing, (s - 1) * kPcStage);
      if (long_split && wv == 0) {  // outside the MFMA work's scheduling groups
        __builtin_amdgcn_sched_barrier(0);
        refill(s);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // a split of one stage took its reference from that stage: no overflow,
    // and both roles skip the test's two barriers
    if (stages <= 1) break;
    m_seen = fmaxf(m_seen, __shfl_xor(m_seen, 16, 64));
    m_seen = fmaxf(m_seen, __shfl_xor(m_seen, 32, 64));
    if (lane < 16) {
      mrg[wv][0][lane] = m_ref;
      mrg[wv][1][lane] = m_seen;
    }
    __syncthreads();
    float mtrue;
    const bool redo = redo_pass(mtrue);
    __syncthreads();
    if (!redo) break;
    m_ref = __shfl(mtrue, col, 64);  // reference: the true max
    if (long_split) {  // as the producers: the first stages' entries again
      build_table();
      wait_vm();
      __syncthreads();
    }
  }

  // ---- finalise this consumer's half of O ----
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);  // sum of the weights of head col against m_ref
  const float mm = m_ref;
  float factor_h, lse_h;
  if (a.ws_splits == 0) {
    const float sink2 = a.sink ? a.sink[head0 + col] * kLog2e : -INFINITY;
    const float mz = fmaxf(mm, sink2);
    factor_h = 0.0f;
    lse_h = -INFINITY;
    if (mz != -INFINITY) {
      const float em = mm == -INFINITY ? 0.0f : exp2f(mm - mz);
      const float z = l_run * em + exp2f(sink2 - mz);
      factor_h = em / z;
      lse_h = (mz + log2f(z)) * kLn2;
    }
    if (half == 0 && lane < 16) a.lse[t * a.heads + head0 + col] = lse_h;
  } else {
    factor_h = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    lse_h = l_run > 0.0f ? mm + log2f(l_run) : -INFINITY;
    if (half == 0 && lane < 16)
      a.ws_lse[(t * a.ws_splits + a.ws_base + split) * a.heads + head0 + col] = lse_h;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * g + i;
    const float f = __shfl(factor_h, h, 64);
    if (a.ws_splits == 0) {
      uint16_t* orow = a.out + (t * a.heads + head0 + h) * kHeadDim + 256 * half + col;
#pragma unroll
      for (int nt = 0; nt < 16; ++nt)
        orow[16 * nt] = __builtin_bit_cast(uint16_t, (__bf16)(o[nt][i] * f));
    } else {
      float* orow = a.ws_o + ((t * a.ws_splits + a.ws_base + split) * a.heads + head0 + h) * kHeadDim +
                    256 * half + col;
      // streaming stores: the partials are read once, by the combine
#pragma unroll
      for (int nt = 0; nt < 16; ++nt) __builtin_nontemporal_store(o[nt][i] * f, orow + 16 * nt);
    }
  }
}

// kLong: splits may run past kPcMaxChunk records (the table ring refill),
// compiled apart so that shorter splits carry none of its code. kPos: the
// RoPE rotation from positions and inverse frequencies instead of table rows.
template <int kHG, bool kPlanes, bool kLong, bool kPos>
__global__ __launch_bounds__((PcRoles<kHG, kTailWaves<true, kHG>>::kThreads)) void
packed_decode_pc_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[sizeof(PcShared<true>)];
  decode_pc<true, kHG, kPlanes, kLong, kPos, kTailWaves<true, kHG>>(
      a, reinterpret_cast<PcShared<true>*>(smem), blockIdx.x);
}
template <int kHG, bool kLong>
__global__ __launch_bounds__(PcRoles<kHG>::kThreads) void native_decode_pc_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[sizeof(PcShared<false>)];
  decode_pc<false, kHG, false, kLong>(a, reinterpret_cast<PcShared<false>*>(smem), blockIdx.x);
}
// C4 list and window rows in one launch: workgroups x < c4.splits take a C4
// split, the last column the window rows (Native records, one short split).
template <bool kPacked, int kHG, bool kPlanes, bool kLong, bool kPos, bool kHelp = false>
__device__ __forceinline__ void decode_joint(const DecodeArgs& c4, const DecodeArgs& swa) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kPcSmemBytes];
  if ((int)blockIdx.x < c4.splits)
    decode_pc<kPacked, kHG, kPlanes, kLong, kPos, kHelp>(
        c4, reinterpret_cast<PcShared<kPacked>*>(smem), blockIdx.x);
  else
    decode_pc<false, kHG, false, false, false, kHelp>(swa, reinterpret_cast<PcShared<false>*>(smem),
                                                      0);
}
template <int kHG, bool kPlanes, bool kLong, bool kPos>
__global__ __launch_bounds__((PcRoles<kHG, kTailWaves<true, kHG>>::kThreads)) void
packed_swa_decode_pc_kernel(DecodeArgs c4, DecodeArgs swa) {
  decode_joint<true, kHG, kPlanes, kLong, kPos, kTailWaves<true, kHG>>(c4, swa);
}
template <int kHG, bool kLong>
__global__ __launch_bounds__(PcRoles<kHG>::kThreads) void native_swa_decode_pc_kernel(
    DecodeArgs c4, DecodeArgs swa) {
  decode_joint<false, kHG, false, kLong, false>(c4, swa);
}

// The workgroup kernel for a format, storage layout, head grouping, split
// length and (Packed) RoPE source.
using SplitKernel = void (*)(DecodeArgs);
using JointKernel = void (*)(DecodeArgs, DecodeArgs);
template <bool kLong, bool kPos>
SplitKernel packed_split_kernel(bool planes, int hg) {
  if (planes)
    return hg == 2 ? packed_decode_pc_kernel<2, true, kLong, kPos>
                   : packed_decode_pc_kernel<1, true, kLong, kPos>;
  return hg == 2 ? packed_decode_pc_kernel<2, false, kLong, kPos>
                 : packed_decode_pc_kernel<1, false, kLong, kPos>;
}
template <bool kPacked, bool kLong>
SplitKernel split_kernel(bool planes, int hg, bool pos) {
  if constexpr (!kPacked)
    return hg == 2 ? native_decode_pc_kernel<2, kLong> : native_decode_pc_kernel<1, kLong>;
  else
    return pos ? packed_split_kernel<kLong, true>(planes, hg)
               : packed_split_kernel<kLong, false>(planes, hg);
}
template <bool kLong, bool kPos>
JointKernel packed_joint_kernel(bool planes, int hg) {
  if (planes)
    return hg == 2 ? packed_swa_decode_pc_kernel<2, true, kLong, kPos>
                   : packed_swa_decode_pc_kernel<1, true, kLong, kPos>;
  return hg == 2 ? packed_swa_decode_pc_kernel<2, false, kLong, kPos>
                 : packed_swa_decode_pc_kernel<1, false, kLong, kPos>;
}
template <bool kPacked, bool kLong>
JointKernel joint_kernel(bool planes, int hg, bool pos) {
  if constexpr (!kPacked)
    return hg == 2 ? native_swa_decode_pc_kernel<2, kLong> : native_swa_decode_pc_kernel<1, kLong>;
  else
    return pos ? packed_joint_kernel<kLong, true>(planes, hg)
               : packed_joint_kernel<kLong, false>(planes, hg);
}

// Butterfly over the wave's 64 lanes with the pairing of xor distances 1, 2,
// 4, ..., 32 (quad permutes, the half-row and row mirrors -- in a butterfly
// every lane of an aligned group already holds the same value, so the mirror
// partner gives the xor partner's value -- then the 16- and 32-lane swaps):
// the same additions as a shuffle-xor butterfly, without LDS round trips.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, false));
}
template <bool kMax>
__device__ __forceinline__ float wave_all(float x) {
  auto op = [](float u, float v) { return kMax ? fmaxf(u, v) : u + v; };
  x = op(x, dpp_f<0xB1>(x));   // quad_perm [1,0,3,2]
  x = op(x, dpp_f<0x4E>(x));   // quad_perm [2,3,0,1]
  x = op(x, dpp_f<0x141>(x));  // row_half_mirror
  x = op(x, dpp_f<0x140>(x));  // row_mirror
  const auto h = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = op(u2f(h[0]), u2f(h[1]));
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return op(u2f(q[0]), u2f(q[1]));
}
__device__ __forceinline__ float lane_of(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

// Merge split partials with the sink, for many rows: one wave per (token,
// head) row, lane l owning coordinates 8l..8l+7. The partial loads of up to
// kWaveBatch splits are issued together with the split LSEs (lane s holds
// split s), so a row costs one round trip per kWaveBatch splits.
constexpr int kWaveBatch = 8;
__global__ __launch_bounds__(256) void combine_wave_kernel(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_lse,
                                                           const float* __restrict__ sink,
                                                           int splits, int64_t heads, int64_t rows,
                                                           uint16_t* __restrict__ out,
                                                           float* __restrict__ lse) {
  const int lane = wave_lane();
  const int64_t row = (int64_t)blockIdx.x * 4 + uniform((int)(threadIdx.x >> 6));
  if (row >= rows) return;
  const int64_t t = row / heads, h = row - t * heads;
  const float* src = ws_o + (t * splits * heads + h) * kHeadDim + 8 * lane;
  const int64_t step = heads * kHeadDim;
  f32x4 x[2 * kWaveBatch];
#pragma unroll
  for (int u = 0; u < kWaveBatch; ++u) {
    x[2 * u] = u < splits ? *(const f32x4*)(src + u * step) : f32x4{0.f, 0.f, 0.f, 0.f};
    x[2 * u + 1] = u < splits ? *(const f32x4*)(src + u * step + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float ls = lane < splits ? ws_lse[(t * splits + lane) * heads + h] : -INFINITY;
  const float sink2 = sink ? sink[h] * kLog2e : -INFINITY;
  const float mz = wave_all<true>(fmaxf(ls, sink2));
  const float w = (mz != -INFINITY && lane < splits) ? exp2f(ls - mz) : 0.0f;
  const float z = wave_all<false>(w);
  f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < splits; s0 += kWaveBatch) {
    if (s0 > 0) {
#pragma unroll
      for (int u = 0; u < kWaveBatch; ++u) {
        const int sp = s0 + u;
        x[2 * u] = sp < splits ? *(const f32x4*)(src + sp * step) : f32x4{0.f, 0.f, 0.f, 0.f};
        x[2 * u + 1] =
            sp < splits ? *(const f32x4*)(src + sp * step + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int u = 0; u < kWaveBatch; ++u) {
      const int sp = s0 + u;
      const float ww = sp < splits ? lane_of(w, sp) : 0.0f;
      a0 += ww * x[2 * u];
      a1 += ww * x[2 * u + 1];
    }
  }
  float lse_out = -INFINITY;
  f32x4 r0 = {0.f, 0.f, 0.f, 0.f}, r1 = {0.f, 0.f, 0.f, 0.f};
  if (mz != -INFINITY) {
    const float zt = z + exp2f(sink2 - mz);
    const float inv = 1.0f / zt;
    r0 = a0 * inv;
    r1 = a1 * inv;
    lse_out = (mz + log2f(zt)) * kLn2;
  }
  *(u32x4*)(out + row * kHeadDim + 8 * lane) =
      u32x4{bf16_rne(r0[0]) | (bf16_rne(r0[1]) << 16), bf16_rne(r0[2]) | (bf16_rne(r0[3]) << 16),
            bf16_rne(r1[0]) | (bf16_rne(r1[1]) << 16), bf16_rne(r1[2]) | (bf16_rne(r1[3]) << 16)};
  if (lane == 0) lse[row] = lse_out;
}

// Merge split partials with the sink, for few rows (small batches). One
// workgroup (4 waves) per (token, head, 64-coordinate slice): lane l owns coordinate 64 slice + l; wave w takes
// splits w, w + 4, ... (<= 16 each, all loads in flight at once); the four
// partial sums meet in LDS in a fixed order. The split weights come from every
// split's LSE, read by every wave (lane s holds split s; splits <= 64).
constexpr int kCombineSlices = kHeadDim / 64;
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ ws_o,
                                                      const float* __restrict__ ws_lse,
                                                      const float* __restrict__ sink, int splits,
                                                      int64_t heads, uint16_t* __restrict__ out,
                                                      float* __restrict__ lse) {
  __shared__ float part[4][64];
  const int lane = wave_lane();
  const int wave = uniform((int)(threadIdx.x >> 6));
  const int64_t row = blockIdx.x / kCombineSlices;
  const int slice = (int)(blockIdx.x - row * kCombineSlices);
  const int64_t t = row / heads, h = row - t * heads;
  const int64_t step = heads * kHeadDim;
  const float* src = ws_o + (t * splits * heads + h) * kHeadDim + 64 * slice + lane;
  // issue every load first: this wave's partials and all split LSEs
  constexpr int kPerWave = kMaxSplits / 4;
  float x[kPerWave];
#pragma unroll
  for (int u = 0; u < kPerWave; ++u) {
    const int s = wave + 4 * u;
    x[u] = s < splits ? src[s * step] : 0.0f;
  }
  const float ls = lane < splits ? ws_lse[(t * splits + lane) * heads + h] : -INFINITY;
  const float sink2 = sink ? sink[h] * kLog2e : -INFINITY;
  const float mz = wave_all<true>(fmaxf(ls, sink2));
  const float w = (mz != -INFINITY && lane < splits) ? exp2f(ls - mz) : 0.0f;
  const float z = wave_all<false>(w);
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kPerWave; ++u) {
    const int s = wave + 4 * u;
    acc += (s < splits ? lane_of(w, s) : 0.0f) * x[u];
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    float lse_out = -INFINITY, r = 0.0f;
    if (mz != -INFINITY) {
      const float zt = z + exp2f(sink2 - mz);
      const float inv = 1.0f / zt;
      r = (part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane]) * inv;
      lse_out = (mz + log2f(zt)) * kLn2;
    }
    out[row * kHeadDim + 64 * slice + lane] = (uint16_t)bf16_rne(r);
    if (lane == 0 && slice == 0) lse[row] = lse_out;
  }
}

struct Plan {
  int splits;
  int chunk;
};

// Split plan: about one workgroup per CU (256 CUs), whole 32-record stages per
// split and at most max_splits splits (the combine merges at most kMaxSplits
// partial slots per row, the window rows' slot included). A split may hold
// more than kPcMaxChunk records (its table ring is refilled as it goes), so
// a batch that fills the round on its own takes one split per token: one
// round of workgroups and no partials to merge.
// 16-head groups per workgroup. Two groups share every expanded record (half
// the expansion work per head) but double a workgroup's consumer work; that
// pays once 16-head workgroups alone would fill the GPU's round of about 256
// workgroups with at most two splits each (measured on the reference's decode
// shapes: H128/B16 27.8 us with two groups vs 33.4 us with one; H128/B8 and
// H64/B8-16 are 10-20 % faster with one).
int head_groups(int64_t tokens, int64_t heads) {
  return heads % (16 * kPcMaxGroups) == 0 && tokens * (heads / 16) >= 128 ? kPcMaxGroups : 1;
}

Plan plan_pc(int64_t tokens, int64_t heads, int64_t topk, int64_t max_splits = kMaxSplits,
             bool window = false) {
  const int64_t base = tokens * (heads / (16 * head_groups(tokens, heads)));
  const int64_t stages = (topk + kPcStage - 1) / kPcStage;
  int64_t splits = base > 0 ? (256 + base - 1) / base : 1;
  // the window rows' workgroups (one per token and head block) share the round
  if (window && base > 0) splits = 256 / base - 1;
  if (splits > stages) splits = stages;
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  int64_t chunk_stages = (stages + splits - 1) / splits;
  if (chunk_stages < 1) chunk_stages = 1;
  splits = (stages + chunk_stages - 1) / chunk_stages;
  if (splits < 1) splits = 1;
  Plan p;
  p.splits = (int)splits;
  p.chunk = (int)(chunk_stages * kPcStage);
  return p;
}

bool aligned(const void* p, uintptr_t al) { return ((uintptr_t)p & (al - 1)) == 0; }

// Sliding-window rows attended jointly with the C4 list: slots of a Native
// pool (64-record pages, tail stored rotated), per token.
struct Swa {
  const uint8_t* pool = nullptr;
  int64_t pool_pages = 0;
  const int32_t* indices = nullptr;  // [tokens, topk] pool slots (-1 = padding)
  int64_t topk = 0;
  const int32_t* length = nullptr;   // [tokens] valid entries (NULL = topk)
};

// Workspace slots per row: the C4 splits, plus one for the window rows.
int64_t ws_slots(const Plan& p, const Swa& w) { return p.splits + (w.topk > 0 ? 1 : 0); }
// C4 splits available next to the window rows' slot.
int64_t c4_max_splits(const Swa& w) { return kMaxSplits - (w.topk > 0 ? 1 : 0); }
size_t ws_bytes(int64_t tokens, int64_t heads, int64_t slots) {
  return slots > 1 ? (size_t)(tokens * slots * heads) * (kHeadDim + 1) * sizeof(float) : 0;
}

// Where the C4 records live: contiguous pages (bitmaps == nullptr) or the
// three planes of `rows` Packed records.
struct Src {
  const uint8_t* pool = nullptr;
  const uint8_t* bitmaps = nullptr;
  const uint8_t* scales = nullptr;
  int64_t pages = 0;
  int64_t rows = 0;
  bool planes() const { return bitmaps != nullptr; }
};
Src paged(const uint8_t* pool, int64_t pages) {
  Src r;
  r.pool = pool;
  r.pages = pages;
  r.rows = pages * kPageRecords;
  return r;
}

template <bool kPacked>
int launch_decode(const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads,
                  const Src& src, const int32_t* block_table,
                  int64_t bt_stride, int64_t max_blocks, const int32_t* seqlens,
                  const int32_t* indices, int64_t topk, const int32_t* topk_length,
                  const Swa& w, const float* sink, const float* freqs, int64_t freq_rows,
                  const float* inv_freq, float scale, uint16_t* out, float* lse,
                  void* workspace, size_t workspace_bytes, void* stream) {
  const uint8_t* pool = src.pool;
  const int64_t pool_pages = src.pages;
  if (batch < 0 || q_len < 0 || topk < 0 || pool_pages < 0 || max_blocks < 0 || freq_rows < 0 ||
      w.topk < 0 || w.pool_pages < 0 || src.rows < 0)
    return RM_ERR_SHAPE;
  // planes: the scale rows of slots 2k and 2k + 1 are copied as one 16-byte piece
  if (src.planes() && (src.rows & 1)) return RM_ERR_SHAPE;
  const int64_t tokens = batch * q_len;
  if (tokens == 0 || heads == 0) return RM_OK;
  if (heads < 0 || heads % 16 || heads > 1024 || bt_stride < max_blocks) return RM_ERR_SHAPE;
  // an invalid record reads frequency row 0 as a stand-in: a table needs one row
  if (kPacked && freqs && freq_rows < 1) return RM_ERR_SHAPE;
  if (topk > (int64_t)kPcMaxChunk * c4_max_splits(w) || w.topk > kPcMaxChunk) return RM_ERR_SHAPE;
  if (pool_pages > ((int64_t)1 << 25) || w.pool_pages > ((int64_t)1 << 25))
    return RM_ERR_SHAPE;  // slots fit in int32
  if (!q || !out || !lse || (topk > 0 && (!indices || !pool || !block_table)) ||
      (w.topk > 0 && (!w.indices || !w.pool)))
    return RM_ERR_NULL;
  if (topk > 0 && src.planes() && !src.scales) return RM_ERR_NULL;
  if (!aligned(q, 16) || !aligned(out, 16) || (pool && !aligned(pool, 16)) ||
      (w.pool && !aligned(w.pool, 16)) || (freqs && !aligned(freqs, 16)) ||
      (inv_freq && !aligned(inv_freq, 16)) ||
      (src.planes() && !(aligned(src.bitmaps, 16) && aligned(src.scales, 16))))
    return RM_ERR_ALIGN;
  if (tokens > 65535) return RM_ERR_SHAPE;
  const Plan plan = plan_pc(tokens, heads, topk, c4_max_splits(w), w.topk > 0);
  const int64_t slots = ws_slots(plan, w);
  const size_t bytes = ws_bytes(tokens, heads, slots);
  if (bytes > 0 && (!workspace || workspace_bytes < bytes)) return RM_ERR_WORKSPACE;
  if (bytes > 0 && !aligned(workspace, 16)) return RM_ERR_ALIGN;
  DecodeArgs a;
  a.q = q;
  a.pool = pool;
  a.bitmaps = src.bitmaps;
  a.scales = src.scales;
  a.pool_pages = pool_pages;
  a.pool_rows = src.rows;
  a.block_table = block_table;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks;
  a.seqlens = seqlens;
  a.indices = indices;
  a.topk = topk;
  a.topk_length = topk_length;
  a.sink = sink;
  a.freqs = kPacked ? freqs : nullptr;
  a.freq_rows = freq_rows;
  a.inv_freq = kPacked ? inv_freq : nullptr;
  // Packed tails rotate from table rows only when a table and no inverse
  // frequencies are given; otherwise by angles computed from the positions
  // (theta = 0, the identity, with neither)
  const bool pos = kPacked && (inv_freq || !freqs);
  a.scale_log2 = scale * kLog2e;
  a.q_len = q_len;
  a.heads = heads;
  a.chunk = plan.chunk;
  a.splits = plan.splits;
  a.ws_splits = slots > 1 ? (int)slots : 0;
  a.ws_base = 0;
  a.out = out;
  a.lse = lse;
  a.ws_o = (float*)workspace;
  a.ws_lse = bytes ? (float*)workspace + (size_t)tokens * slots * heads * kHeadDim : nullptr;
  hipStream_t s = (hipStream_t)stream;
  const int hg = head_groups(tokens, heads);
  // (Packed decodes at 16 heads add the tail waves)
  const dim3 block(hg == 2    ? PcRoles<2>::kThreads
                   : kPacked ? PcRoles<1, true>::kThreads
                             : PcRoles<1>::kThreads);
  const unsigned zblocks = (unsigned)(heads / (16 * hg));
  const bool lng = plan.chunk > kPcMaxChunk;
  if (w.topk > 0) {
    // the window rows are one more split, read by the Native path of the same launch
    DecodeArgs b = a;
    b.pool = w.pool;
    b.bitmaps = nullptr;
    b.scales = nullptr;
    b.pool_pages = w.pool_pages;
    b.pool_rows = w.pool_pages * kPageRecords;
    b.block_table = nullptr;  // entries are pool slots
    b.seqlens = nullptr;
    b.indices = w.indices;
    b.topk = w.topk;
    b.topk_length = w.length;
    b.freqs = nullptr;
    b.freq_rows = 0;
    b.inv_freq = nullptr;
    b.chunk = kPcMaxChunk;
    b.splits = 1;
    b.ws_base = plan.splits;
    const dim3 grid((unsigned)slots, (unsigned)tokens, zblocks);
    const JointKernel kern = lng ? joint_kernel<kPacked, true>(src.planes(), hg, pos)
                                 : joint_kernel<kPacked, false>(src.planes(), hg, pos);
    hipLaunchKernelGGL(kern, grid, block, 0, s, a, b);
  } else {
    const dim3 grid((unsigned)plan.splits, (unsigned)tokens, zblocks);
    const SplitKernel kern = lng ? split_kernel<kPacked, true>(src.planes(), hg, pos)
                                 : split_kernel<kPacked, false>(src.planes(), hg, pos);
    hipLaunchKernelGGL(kern, grid, block, 0, s, a);
  }
  if (hipGetLastError() != hipSuccess) return RM_ERR_LAUNCH;
  if (slots > 1) {
    const int64_t rows = tokens * heads;
    if (rows < 256)  // too few rows to fill the GPU: one workgroup per 64 coordinates
      hipLaunchKernelGGL(combine_kernel, dim3((unsigned)(rows * kCombineSlices)), dim3(256), 0, s,
                         a.ws_o, a.ws_lse, sink, (int)slots, heads, out, lse);
    else
      hipLaunchKernelGGL(combine_wave_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s,
                         a.ws_o, a.ws_lse, sink, (int)slots, heads, rows, out, lse);
    if (hipGetLastError() != hipSuccess) return RM_ERR_LAUNCH;
  }
  return RM_OK;
}

}  // namespace

extern "C" int rm_sparse_decode_workspace(int64_t tokens, int64_t heads, int64_t topk,
                                          int32_t* num_splits, size_t* workspace_bytes) {
  return rm_sparse_decode_workspace_swa(tokens, heads, topk, 0, num_splits, workspace_bytes);
}

extern "C" int rm_sparse_decode_workspace_swa(int64_t tokens, int64_t heads, int64_t topk,
                                              int64_t swa_topk, int32_t* num_splits,
                                              size_t* workspace_bytes) {
  Swa w;
  w.topk = swa_topk;
  if (tokens < 0 || heads < 0 || heads % 16 || topk < 0 || swa_topk < 0 ||
      swa_topk > kPcMaxChunk || topk > (int64_t)kPcMaxChunk * c4_max_splits(w))
    return RM_ERR_SHAPE;
  const Plan p = plan_pc(tokens, heads, topk, c4_max_splits(w), w.topk > 0);
  const int64_t slots = ws_slots(p, w);
  if (num_splits) *num_splits = (int32_t)slots;
  if (workspace_bytes) *workspace_bytes = ws_bytes(tokens, heads, slots);
  return RM_OK;
}

extern "C" int rm_remnant_sparse_decode_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* pool,
    int64_t pool_pages, const int32_t* block_table, int64_t block_table_stride,
    int64_t max_blocks, const int32_t* seqlens, const int32_t* indices, int64_t topk,
    const int32_t* topk_length, const float* sink, const float* freqs, int64_t freq_rows,
    const float* inv_freq, float softmax_scale, uint16_t* out, float* lse, void* workspace,
    size_t workspace_bytes, void* stream) {
  return launch_decode<true>(q, batch, q_len, heads, paged(pool, pool_pages), block_table,
                             block_table_stride, max_blocks, seqlens, indices, topk, topk_length,
                             Swa(), sink, freqs, freq_rows, inv_freq, softmax_scale, out, lse,
                             workspace, workspace_bytes, stream);
}

namespace {

// ---- allocation-free variant ----
// The split partials of rm_remnant_sparse_decode_swa_noalloc_fwd live in this
// file-scope device array instead of a caller workspace. Each GPU the library
// runs on holds its own copy until the process ends. In host code `scratch`
// names a host-side stand-in, never the device array: its device address is
// looked up once per device -- the device of the call's stream -- by
// hipGetSymbolAddress with that device current, on the first call there (so a
// caller that captures the call in a HIP graph makes one eager call on that
// device first), and only that address reaches kernels. Every split writes its
// whole partial slot before the combine reads it, so nothing needs clearing
// between calls; calls that overlap on one GPU share the array and race.
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device of `stream` (the current device
// for the null stream); nullptr on failure.
void* scratch_address(hipStream_t stream) {
  int cur = -1, dev = -1;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  dev = cur;
  if (stream && hipStreamGetDevice(stream, &dev) != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (dev != cur && hipSetDevice(dev) != hipSuccess) return nullptr;
    const hipError_t st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur && hipSetDevice(cur) != hipSuccess) return nullptr;
    if (st != hipSuccess) return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int rm_remnant_sparse_decode_swa_noalloc_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* pool,
    int64_t pool_pages, const int32_t* block_table, int64_t block_table_stride,
    int64_t max_blocks, const int32_t* seqlens, const int32_t* indices, int64_t topk,
    const int32_t* topk_length, const uint8_t* swa_pool, int64_t swa_pool_pages,
    const int32_t* swa_indices, int64_t swa_topk, const int32_t* swa_length, const float* sink,
    const float* freqs, int64_t freq_rows, const float* inv_freq, float softmax_scale,
    uint16_t* out, float* lse, void* stream) {
  // a partial slot set beyond the array is refused before any launch
  int32_t splits = 0;
  size_t need = 0;
  const int st = rm_sparse_decode_workspace_swa(batch * q_len, heads, topk, swa_topk, &splits,
                                                &need);
  if (st != RM_OK) return st;
  if (need > kScratchBytes) return RM_ERR_WORKSPACE;
  void* ws = nullptr;
  if (need > 0 && !(ws = scratch_address((hipStream_t)stream))) return RM_ERR_LAUNCH;
  return rm_remnant_sparse_decode_swa_fwd(q, batch, q_len, heads, pool, pool_pages, block_table,
                                          block_table_stride, max_blocks, seqlens, indices, topk,
                                          topk_length, swa_pool, swa_pool_pages, swa_indices,
                                          swa_topk, swa_length, sink, freqs, freq_rows, inv_freq,
                                          softmax_scale, out, lse, ws, need, stream);
}

extern "C" int rm_remnant_sparse_decode_swa_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* pool,
    int64_t pool_pages, const int32_t* block_table, int64_t block_table_stride,
    int64_t max_blocks, const int32_t* seqlens, const int32_t* indices, int64_t topk,
    const int32_t* topk_length, const uint8_t* swa_pool, int64_t swa_pool_pages,
    const int32_t* swa_indices, int64_t swa_topk, const int32_t* swa_length, const float* sink,
    const float* freqs, int64_t freq_rows, const float* inv_freq, float softmax_scale,
    uint16_t* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  Swa w;
  w.pool = swa_pool;
  w.pool_pages = swa_pool_pages;
  w.indices = swa_indices;
  w.topk = swa_topk;
  w.length = swa_length;
  return launch_decode<true>(q, batch, q_len, heads, paged(pool, pool_pages), block_table,
                             block_table_stride, max_blocks, seqlens, indices, topk, topk_length,
                             w, sink, freqs, freq_rows, inv_freq, softmax_scale, out, lse,
                             workspace, workspace_bytes, stream);
}

extern "C" int rm_remnant_sparse_decode_planes_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* values,
    const uint64_t* bitmaps, const uint8_t* scales, int64_t pool_rows,
    const int32_t* block_table, int64_t block_table_stride, int64_t max_blocks,
    const int32_t* seqlens, const int32_t* indices, int64_t topk, const int32_t* topk_length,
    const uint8_t* swa_pool, int64_t swa_pool_pages, const int32_t* swa_indices,
    int64_t swa_topk, const int32_t* swa_length, const float* sink, const float* freqs,
    int64_t freq_rows, const float* inv_freq, float softmax_scale, uint16_t* out, float* lse,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (pool_rows < 0 || pool_rows > ((int64_t)1 << 31)) return RM_ERR_SHAPE;
  if (!bitmaps && topk > 0) return RM_ERR_NULL;
  Src src;
  src.pool = values;
  src.bitmaps = (const uint8_t*)bitmaps;
  src.scales = scales;
  src.rows = pool_rows;
  src.pages = (pool_rows + kPageRecords - 1) / kPageRecords;
  if (!bitmaps) src = paged(values, 0);  // nothing is read
  Swa w;
  w.pool = swa_pool;
  w.pool_pages = swa_pool_pages;
  w.indices = swa_indices;
  w.topk = swa_topk;
  w.length = swa_length;
  return launch_decode<true>(q, batch, q_len, heads, src, block_table, block_table_stride,
                             max_blocks, seqlens, indices, topk, topk_length, w, sink, freqs,
                             freq_rows, inv_freq, softmax_scale, out, lse, workspace,
                             workspace_bytes, stream);
}

extern "C" int rm_native_sparse_decode_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* pool,
    int64_t pool_pages, const int32_t* block_table, int64_t block_table_stride,
    int64_t max_blocks, const int32_t* seqlens, const int32_t* indices, int64_t topk,
    const int32_t* topk_length, const float* sink, float softmax_scale, uint16_t* out,
    float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  return launch_decode<false>(q, batch, q_len, heads, paged(pool, pool_pages), block_table,
                              block_table_stride, max_blocks, seqlens, indices, topk,
                              topk_length, Swa(), sink, nullptr, 0, nullptr, softmax_scale, out,
                              lse, workspace, workspace_bytes, stream);
}

extern "C" int rm_native_sparse_decode_swa_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* pool,
    int64_t pool_pages, const int32_t* block_table, int64_t block_table_stride,
    int64_t max_blocks, const int32_t* seqlens, const int32_t* indices, int64_t topk,
    const int32_t* topk_length, const uint8_t* swa_pool, int64_t swa_pool_pages,
    const int32_t* swa_indices, int64_t swa_topk, const int32_t* swa_length, const float* sink,
    float softmax_scale, uint16_t* out, float* lse, void* workspace, size_t workspace_bytes,
    void* stream) {
  Swa w;
  w.pool = swa_pool;
  w.pool_pages = swa_pool_pages;
  w.indices = swa_indices;
  w.topk = swa_topk;
  w.length = swa_length;
  return launch_decode<false>(q, batch, q_len, heads, paged(pool, pool_pages), block_table,
                              block_table_stride, max_blocks, seqlens, indices, topk,
                              topk_length, w, sink, nullptr, 0, nullptr, softmax_scale, out, lse,
                              workspace, workspace_bytes, stream);
}

extern "C" int rm_version(void) { return 300; }
