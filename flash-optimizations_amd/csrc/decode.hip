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
// Work split. One workgroup of four waves owns (split, token, 16-head block) and
// walks its share of the top-k list in tiles of 16 records:
//   * record metadata (index -> block table -> page/row, validity) for the
//     share (<= 256 records) is resolved once into LDS;
//   * the next tile's record bytes and RoPE rows are copied HBM -> LDS with
//     global_load_lds while the current tile computes (double-buffered);
//   * wave w owns coordinates 16w .. 16w+15 of every 64-coordinate word (a
//     128-coordinate slice, the tail word included, so RoPE work is balanced):
//     it dequantizes only its slice -- v_perm places the kept E4M3 codes
//     (zeros for pruned coordinates) from a 256-entry selector table,
//     v_cvt_scalef32_pk_bf16_fp8 applies the UE8M0 scale, tail pairs are
//     BF16-rounded then rotated -- into a wave-private BF16 K slice in LDS;
//   * partial S^T = K Q^T over the slice on v_mfma_f32_16x16x32_bf16 (Q slice in
//     registers); the four partials are summed through LDS (one barrier);
//   * softmax in the log2 domain against a fixed per-head reference (the first
//     valid tile's max), so O is never rescaled inside the loop; weights up to
//     2^64 are far inside FP32/BF16 range, and a split whose scores climb higher
//     is recomputed once against its true max;
//   * O[:, slice] += P K_slice on v_mfma_f32_16x16x16_bf16: P is the S^T
//     accumulator itself, K is read with ds_read_b64_tr_b16 (4 records of one
//     coordinate per lane); O stays in accumulator registers.
// A split count > 1 writes (O/l, m + log2 l) partials merged with the sink by a
// combine kernel; a single split finalises in place.
#include <type_traits>

#include "remnant_device.h"
#include "remnant_mi355x.h"

using namespace rm;

namespace {

constexpr int kT = 16;                     // records per tile
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kSlicePitch = 128 + 8;       // BF16 per K-slice row (272 B, 16-B aligned)
constexpr int kMaxChunk = 240;             // records per split (five three-tile groups)
constexpr int kMaxSplits = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr uint64_t kAddrMask = (1ull << 58) - 1;
constexpr float kRefSlack = 64.0f;         // log2 headroom above the reference max

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

struct DecodeArgs {
  const uint16_t* q;
  const uint8_t* pool;
  int64_t pool_pages;
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
  float scale_log2;
  int64_t q_len;
  int64_t heads;
  int chunk;       // records per split (multiple of kT, <= kMaxChunk)
  int splits;
  uint16_t* out;
  float* lse;
  float* ws_o;     // [tokens, splits, heads, 512]
  float* ws_lse;   // [tokens, splits, heads]
};

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return bf16_rne(a) | (bf16_rne(b) << 16);
}

// Two E4M3 codes (bytes 0-1, or 2-3 with kHi) times scale -> two BF16 (exact).
template <bool kHi>
__device__ __forceinline__ uint32_t cvt2(uint32_t codes, float scale) {
  bf16x2 r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(codes, scale, kHi);
  return __builtin_bit_cast(uint32_t, r);
}

// Staging geometry. Tiles are copied HBM -> LDS with global_load_lds (lane i
// of a 16-byte copy fills bytes 16 i .. 16 i + 15 of a 1 KiB run), so a tile
// lands as consecutive 16-byte pieces: piece c of the tile (record c / kPieces,
// piece c % kPieces) goes to staging byte 16 c.
// A Packed record (328 B, 8-byte aligned) is fetched as the 21 aligned 16-byte
// pieces covering it: an even pool row from its start (its last piece reaches 8
// bytes into the next row of the same page, which always exists because row 63
// is odd), an odd row from 8 bytes before it, so it sits at staging offset 8.
// A Native record stages its 576-byte data row (36 pieces); its scale row goes
// to an 8-byte slot after the rows (4-byte copies, two per record).
// Every wave issues the same, fixed number of copies per tile and every lane of
// a copy is active -- lanes without a record of the tile read a harmless
// source and land in slack bytes or a junk run -- so the wait counts in the
// tile loop are compile-time constants. Invalid records are masked to zero in
// the dequantization, which keeps K finite so that P = 0 removes them exactly.
template <bool kPacked>
struct Geo {
  static constexpr int kData = kPacked ? kRecordBytes : kNativeDataBytes;  // pool row pitch
  static constexpr int kPage = kPacked ? kPageBytes : kNativePageBytes;
  static constexpr int kPieces = kPacked ? 21 : kNativeDataBytes / 16;
  static constexpr int kStage = 16 * kPieces;                 // staging row pitch
  static constexpr int kChunks = kT * kPieces;
  static constexpr int kLoads = (kChunks + 63) / 64;          // 1 KiB runs holding the tile
  static constexpr int kPerWave = (kLoads + kWaves - 1) / kWaves;
  static constexpr int kScaleAt = 1024 * kLoads;              // Native: 64 lanes x 4 B
  static constexpr int kBytes = kScaleAt + (kPacked ? 0 : 256);
  // global loads per wave per tile: kPerWave 16-byte copies, plus the RoPE values
  // (Packed, into registers) or one 4-byte scale copy (Native)
  static constexpr int kWaveLoads = kPerWave + 1;
};

typedef __attribute__((address_space(3))) void lds_void;

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

// Exclusive prefix sum of x over the 4 lanes of a quad (lanes 4k .. 4k+3).
__device__ __forceinline__ int quad_exclusive_sum(int x, int u) {
  // quad_perm(0,0,1,2): lane u reads lane u-1; quad_perm(0,0,0,1): lane u reads lane u-2
  const int t1 = __builtin_amdgcn_mov_dpp(x, 0x90, 0xf, 0xf, false);
  const int s1 = x + (u >= 1 ? t1 : 0);
  const int t2 = __builtin_amdgcn_mov_dpp(s1, 0x40, 0xf, 0xf, false);
  const int s2 = s1 + (u >= 2 ? t2 : 0);
  return s2 - x;
}

template <bool kPacked>
__device__ __forceinline__ void decode_split(const DecodeArgs& a) {
  using G = Geo<kPacked>;
  // staging (double-buffered, row kT zero), per-wave K slices, S partials, tables
  __shared__ __attribute__((aligned(16))) uint8_t stage0[G::kBytes];
  __shared__ __attribute__((aligned(16))) uint8_t stage1[G::kBytes];
  __shared__ __attribute__((aligned(16))) uint8_t stage2[G::kBytes];
  __shared__ __attribute__((aligned(16))) uint8_t junk[1024];  // target of padding copies
  __shared__ __attribute__((aligned(16))) uint16_t kq[kWaves][kT * kSlicePitch];
  __shared__ __attribute__((aligned(16))) f32x4 spart[kWaves][64];
  __shared__ __attribute__((aligned(16))) uint64_t sel_tab[kPacked ? 256 : 1];
  // per record of the split: pool address of its row (0 = invalid record; Native
  // entries carry the row-in-page in bits 58..63, above any virtual address),
  // and for Packed the address of its RoPE row
  __shared__ uint64_t row_tab[kMaxChunk];
  __shared__ uint64_t aux_tab[kPacked ? kMaxChunk : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);  // wave: owns coordinates 16w .. 16w+15 of every word
  const int g = lane >> 4, col = lane & 15;
  const int split = blockIdx.x;
  const int64_t t = blockIdx.y;
  const int64_t head0 = (int64_t)blockIdx.z * 16;
  const int64_t b = t / a.q_len;

  int64_t len = a.topk;
  if (a.topk_length) {
    const int64_t l = a.topk_length[t];
    len = l < 0 ? 0 : (l < a.topk ? l : a.topk);
  }
  const int64_t k0 = (int64_t)split * a.chunk;
  const int64_t k1 = k0 + a.chunk < len ? k0 + a.chunk : len;
  const int n = k1 > k0 ? (int)(k1 - k0) : 0;
  const int64_t seqlen = a.seqlens ? a.seqlens[b] : INT64_MAX;

  // ---- setup: zero rows, selectors, record metadata, Q slice ----
  if (kPacked) {
    // byte bits MSB-first = coordinates 0..7; selector byte i = rank of i or 0x0c (zero)
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
  for (int i = tid; i < n; i += kThreads) {
    const int64_t r = a.indices[t * a.topk + k0 + i];
    bool ok = r >= 0 && r < seqlen && (r >> 6) < a.max_blocks;
    const int64_t page = ok ? a.block_table[b * a.bt_stride + (r >> 6)] : -1;
    ok = ok && page >= 0 && page < a.pool_pages;
    if (kPacked && a.freqs) ok = ok && r * 4 < a.freq_rows;
    const uint8_t* pg = a.pool + (ok ? page : 0) * G::kPage;
    row_tab[i] = ok ? (uint64_t)(pg + (r & 63) * G::kData) | (kPacked ? 0 : (uint64_t)(r & 63) << 58)
                    : 0;
    if (kPacked) aux_tab[i] = (uint64_t)(a.freqs ? a.freqs + (ok ? r : 0) * 4 * 64 : nullptr);
  }
  // B operand of S^T = K Q^T over this wave's 128 coordinates: k-step ks covers
  // slice positions 32 ks .. 32 ks + 31 = coordinates 16w .. 16w+15 of words
  // 2 ks and 2 ks + 1; lane (g, col) holds Q[head col][slice 32 ks + 8 g .. +7].
  bf16x8 qreg[4];
  {
    const uint16_t* qh = a.q + (t * a.heads + head0 + col) * kHeadDim;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int coord = 64 * (2 * ks + (g >> 1)) + 16 * w + 8 * (g & 1);
      qreg[ks] = __builtin_bit_cast(bf16x8, *(const u32x4*)(qh + coord));
    }
  }
  f32x4 o[8];  // O[head 4g + i][coord 64 nt + 16 w + col]
  // Softmax state of head col (log2 domain, identical in every wave): weights
  // are taken against a fixed reference m_ref -- the first valid tile's max --
  // so O is never rescaled inside the loop; l_run sums them, m_seen tracks the
  // true max.
  float m_ref = -INFINITY, m_seen = -INFINITY, l_run = 0.0f;
  wait_vm();  // Q in registers before the tile loop (keeps its waits static)
  __syncthreads();

  // ---- tile copy HBM -> LDS staging (asynchronous). Wave w issues the copies
  // j = w, w + 4, ... and, for Packed, loads into registers the RoPE values its
  // lanes apply (lane (r, u): pairs 8w + 2u, 8w + 2u + 1 of record r). ----
  const uint8_t* const dummy = (const uint8_t*)a.q;  // any readable 16-byte-aligned bytes
  const uint32_t stage_at[3] = {lds_addr(stage0), lds_addr(stage1), lds_addr(stage2)};
  const uint32_t junk_at = lds_addr(junk);
  f32x4 fq0 = {0.f, 0.f, 0.f, 0.f}, fq1 = fq0, fq2 = fq0;
  auto issue_tile = [&](int base, auto buf) {
    constexpr int kB = decltype(buf)::value;
#pragma unroll
    for (int jj = 0; jj < G::kPerWave; ++jj) {
      const int j = jj * kWaves + w;  // this wave's run; runs >= kLoads are padding
      const int c = lane + 64 * j;
      const int r = c / G::kPieces, piece = c - r * G::kPieces;
      const uint64_t row = c < G::kChunks && base + r < n ? row_tab[base + r] : 0;
      // Packed rows are fetched from their 16-byte-aligned start (8 bytes early
      // for odd rows)
      const uint8_t* src =
          row ? (const uint8_t*)(row & (kPacked ? ~(uint64_t)15 : kAddrMask)) + 16 * piece : dummy;
      dma16(src, j < G::kLoads ? stage_at[kB] + 1024 * j : junk_at);
    }
    if (kPacked) {
      const int r = lane >> 2, u = lane & 3;
      const uint64_t row = base + r < n ? row_tab[base + r] : 0;
      const float* src = row && a.freqs ? (const float*)aux_tab[base + r] + 16 * w + 4 * u
                                        : (const float*)dummy;
      // a global (not flat) load: flat loads also count against the LDS counter
      const f32x4 v = *(const __attribute__((address_space(1))) f32x4*)src;
      if (kB == 0) fq0 = v; else if (kB == 1) fq1 = v; else fq2 = v;
    } else {
      // scale rows: lane 2r + h copies bytes 4h .. 4h + 3 of record r's (wave 3;
      // the other waves pad)
      const int r = lane >> 1;
      const uint64_t row = w == kWaves - 1 && lane < 2 * kT && base + r < n ? row_tab[base + r] : 0;
      const uint32_t rip = (uint32_t)(row >> 58);  // row in page
      const uint8_t* src = row ? (const uint8_t*)(row & kAddrMask) - rip * G::kData +
                                     kPageRecords * G::kData + rip * kScaleBytes + 4 * (lane & 1)
                               : dummy;
      dma4(src, w == kWaves - 1 ? stage_at[kB] + G::kScaleAt : junk_at);
    }
  };

  uint16_t* const slice = kq[w];
  // ---- one tile: dequantize this wave's slice, S partial, exchange, softmax, PV ----
  auto compute_tile = [&](int base, const uint8_t* stage, const f32x4 fqv) {
    // lane (record r = lane/4, u = lane%4) expands coordinates 16w .. 16w+15 of
    // words 2u and 2u+1 into slice positions 16 word .. 16 word + 15
    const int r = lane >> 2, u = lane & 3;
    const uint64_t rowaddr = base + r < n ? row_tab[base + r] : 0;
    const bool valid = rowaddr != 0;
    uint16_t* srow = slice + r * kSlicePitch;
    if (kPacked) {
      const uint8_t* st = stage + r * G::kStage + ((uint32_t)rowaddr & 8u);  // odd rows: +8
      // an invalid record reads as an all-pruned bitmap with zero scales
      const u32x2 b0 = *(const u32x2*)(st + kCodeBytes + 16 * u);
      const u32x2 b1 = *(const u32x2*)(st + kCodeBytes + 16 * u + 8);
      const uint64_t wd[2] = {valid ? ((uint64_t)b0[1] << 32) | b0[0] : 0ull,
                              valid ? ((uint64_t)b1[1] << 32) | b1[0] : 0ull};
      // scale bytes of words 2u, 2u+1 (one 32-bit word of the 8 scale bytes)
      const uint32_t sb = valid ? *(const uint32_t*)(st + kDataBytes + 4 * (u >> 1)) : 0u;
      const int c0 = __popcll(wd[0]);
      int rank_word = quad_exclusive_sum(c0 + __popcll(wd[1]), u);  // codes before word 2u
      const uint64_t before = ~(~0ull >> (16 * w));  // coordinates before 16w in a word
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int word = 2 * u + h2;
        const uint64_t bits = wd[h2];
        const float scale = exp2i((int)((sb >> (8 * (word & 3))) & 0xffu) - 127);
        const uint32_t two = (uint32_t)(bits >> (48 - 16 * w)) & 0xffffu;  // chunks 2w, 2w+1
        int rank = rank_word + __popcll(bits & before);
        rank_word += h2 == 0 ? c0 : 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t byte = h == 0 ? two >> 8 : two & 0xffu;
          const uint32_t* cw = (const uint32_t*)(st + (rank & ~3));
          const uint32_t d0 = cw[0], d1 = cw[1], d2 = cw[2];
          // v_alignbyte uses the low two bits of its shift operand only
          const uint32_t lo4 = __builtin_amdgcn_alignbyte(d1, d0, (uint32_t)rank);
          const uint32_t hi4 = __builtin_amdgcn_alignbyte(d2, d1, (uint32_t)rank);
          const uint64_t sel = sel_tab[byte];
          const uint32_t lo = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)sel);
          const uint32_t hi = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)(sel >> 32));
          rank += __popc(byte);
          u32x4 v = {cvt2<false>(lo, scale), cvt2<true>(lo, scale), cvt2<false>(hi, scale),
                     cvt2<true>(hi, scale)};
          *(u32x4*)(srow + 16 * word + 8 * h) = v;
        }
      }
    } else {
      // an invalid record reads as zero codes, zero tail and zero scales
      const uint8_t* st = stage + r * G::kStage;
      const uint32_t sb =
          valid ? *(const uint32_t*)(stage + G::kScaleAt + r * kScaleBytes + 4 * (u >> 1)) : 0u;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int word = 2 * u + h2;
        if (h2 == 0 || u < 3) {
          const float scale = exp2i((int)((sb >> (8 * (word & 3))) & 0xffu) - 127);
          const u32x4 raw = *(const u32x4*)(st + 64 * word + 16 * w);
          const u32x4 codes = valid ? raw : u32x4{0u, 0u, 0u, 0u};
          *(u32x4*)(srow + 16 * word) = u32x4{cvt2<false>(codes[0], scale), cvt2<true>(codes[0], scale),
                                              cvt2<false>(codes[1], scale), cvt2<true>(codes[1], scale)};
          *(u32x4*)(srow + 16 * word + 8) = u32x4{cvt2<false>(codes[2], scale), cvt2<true>(codes[2], scale),
                                                  cvt2<false>(codes[3], scale), cvt2<true>(codes[3], scale)};
        } else {  // tail word: rotated BF16 as stored
          const u32x4 t0 = *(const u32x4*)(st + kNopeDim + 32 * w);
          const u32x4 t1 = *(const u32x4*)(st + kNopeDim + 32 * w + 16);
          *(u32x4*)(srow + 16 * word) = valid ? t0 : u32x4{0u, 0u, 0u, 0u};
          *(u32x4*)(srow + 16 * word + 8) = valid ? t1 : u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
    if (kPacked && a.freqs) {
      // tail word: rotate this wave's 8 (re, im) pairs per record with the
      // record's RoPE values; lane (r, u) takes pairs 2u and 2u+1 of record r
      wave_lds_sync();
      const f32x4 cs4 = valid ? fqv : f32x4{0.f, 0.f, 0.f, 0.f};
      uint16_t* tail = srow + 16 * 7 + 4 * u;
      const u32x2 v = *(const u32x2*)tail;
      float x[4] = {u2f(v[0] << 16), u2f(v[0] & 0xffff0000u), u2f(v[1] << 16),
                    u2f(v[1] & 0xffff0000u)};
      const float xr0 = x[0] * cs4[0], xi0 = x[1] * cs4[1], xs0 = x[0] * cs4[1], xc0 = x[1] * cs4[0];
      const float xr1 = x[2] * cs4[2], xi1 = x[3] * cs4[3], xs1 = x[2] * cs4[3], xc1 = x[3] * cs4[2];
      const bf16x4 rot = {(__bf16)(xr0 - xi0), (__bf16)(xs0 + xc0), (__bf16)(xr1 - xi1),
                          (__bf16)(xs1 + xc1)};
      *(bf16x4*)tail = rot;
    }
    // validity of the tile's records: bit 4r of vball
    const uint64_t vball = __ballot(valid);
    wave_lds_sync();  // slice complete (read by this wave only)

    // partial S^T[rec][head] over this wave's coordinates
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    {
      const uint16_t* kr = slice + col * kSlicePitch + 8 * g;
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, *(const u32x4*)kr), qreg[0], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, *(const u32x4*)(kr + 32)), qreg[1], s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, *(const u32x4*)(kr + 64)), qreg[2], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, *(const u32x4*)(kr + 96)), qreg[3], s1, 0, 0, 0);
    }
    spart[w][lane] = s0 + s1;
    block_sync_lds();  // all four partials written
    const f32x4 sacc = spart[0][lane] + spart[1][lane] + spart[2][lane] + spart[3][lane];

    // Softmax against the fixed reference (lane holds S^T[rec 4g + i][head col]).
    // Weight sums and the running max stay per lane (4 records each) and are
    // reduced across the wave once, after the loop.
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool v = (vball >> (4 * (4 * g + i))) & 1u;
      sv[i] = v ? sacc[i] * a.scale_log2 : -INFINITY;
      m_seen = fmaxf(m_seen, sv[i]);
    }
    if (m_ref == -INFINITY) {  // until the first tile with a valid record (wave-uniform)
      float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      m_ref = mt;
    }
    const float mr = m_ref == -INFINITY ? 0.0f : m_ref;  // no valid record yet: all weights 0
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = __builtin_amdgcn_exp2f(sv[i] - mr);
      l_run += p[i];
    }

    // O[head][coord] += P[head][rec] K[rec][coord] over this wave's 8 column blocks;
    // lane (g, j = col) points at K[4g + j/4][block + 4(j%4)] and receives
    // K[4g + 0..3][block + j] (transpose read)
    const bf16x4 pb = {(__bf16)p[0], (__bf16)p[1], (__bf16)p[2], (__bf16)p[3]};
    const s16x4 pa = __builtin_bit_cast(s16x4, pb);
    const uint16_t* kr = slice + (4 * g + (col >> 2)) * kSlicePitch + 4 * (col & 3);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const s16x4 kb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(kr + 16 * nt));
      o[nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, kb, o[nt], 0, 0, 0);
    }
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) asm volatile("" : "+a"(o[nt]));  // O stays in place
    wave_lds_sync();  // slice reads done before the next dequantization
  };

  // Pass 0 runs with m_ref from the first valid tile. If a later score exceeds it
  // by more than 2^kRefSlack (weights, O and l_run could then leave the safe
  // FP32/BF16 range), the split is recomputed once with m_ref = the true max,
  // which bounds every weight by 1. Otherwise the result is exact up to
  // rounding: the final normalisation divides the common factor out. The
  // decision depends on S only, so every wave takes the same path.
  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      asm volatile("" : "+a"(o[nt]));  // O lives in accumulator registers
    }
    l_run = 0.0f;
    // Tile i is staged in buffer i % 3; its copy is issued two tiles ahead, so
    // it overlaps the computation of the two tiles before it. The loop runs
    // whole groups of three tiles (tiles past n are empty: their copies read a
    // harmless source and every record is masked), so each step issues the same
    // loads and the wait counts are static.
    auto step = [&](int tb, auto buf) {
      constexpr int kB = decltype(buf)::value;
      // this wave's loads for tile tb are complete once at most those of tile
      // tb + kT (issued after them) remain outstanding
      wait_vm_upto<G::kWaveLoads>();
      block_sync_lds();  // tile tb staged by every wave; buffer (kB + 2) % 3 is free
      issue_tile(tb + 2 * kT, std::integral_constant<int, (kB + 2) % 3>{});
      if (kB == 0) compute_tile(tb, stage0, fq0);
      else if (kB == 1) compute_tile(tb, stage1, fq1);
      else compute_tile(tb, stage2, fq2);
    };
    if (n > 0) {
      issue_tile(0, std::integral_constant<int, 0>{});
      issue_tile(kT, std::integral_constant<int, 1>{});
    }
    for (int base = 0; base < n; base += 3 * kT) {
      step(base, std::integral_constant<int, 0>{});
      step(base + kT, std::integral_constant<int, 1>{});
      step(base + 2 * kT, std::integral_constant<int, 2>{});
    }
    wait_vm();  // drain the copies issued for tiles past the end
    m_seen = fmaxf(m_seen, __shfl_xor(m_seen, 16, 64));
    m_seen = fmaxf(m_seen, __shfl_xor(m_seen, 32, 64));
    if (!__ballot(m_seen > m_ref + kRefSlack)) break;
    m_ref = m_seen;
    __syncthreads();  // staging and partials are reused by the second pass
  }
  const float m_run = m_ref;
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  // lane holds O[head 4g + i][coord 64 nt + 16 w + col]; softmax state of head col

  if (a.splits == 1) {
    const float sink2 = a.sink ? a.sink[head0 + col] * kLog2e : -INFINITY;
    const float mz = fmaxf(m_run, sink2);
    float factor = 0.0f, lse = -INFINITY;
    if (mz != -INFINITY) {
      const float em = exp2f(m_run - mz);
      const float z = l_run * em + exp2f(sink2 - mz);
      factor = em / z;
      lse = (mz + log2f(z)) * kLn2;
    }
    if (w == 0 && lane < 16) a.lse[t * a.heads + head0 + col] = lse;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = __shfl(factor, 4 * g + i, 64);
      uint16_t* orow = a.out + (t * a.heads + head0 + 4 * g + i) * kHeadDim + 16 * w + col;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) orow[64 * nt] = __builtin_bit_cast(uint16_t, (__bf16)(o[nt][i] * f));
    }
  } else {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const float plse = l_run > 0.0f ? m_run + log2f(l_run) : -INFINITY;
    const int64_t slot = (t * a.splits + split) * a.heads + head0;
    if (w == 0 && lane < 16) a.ws_lse[slot + col] = plse;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = __shfl(inv, 4 * g + i, 64);
      float* orow = a.ws_o + (slot + 4 * g + i) * kHeadDim + 16 * w + col;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) orow[64 * nt] = o[nt][i] * f;
    }
  }
}

// One kernel per format. Both run three workgroups (12 waves) per CU; the
// Native body needs a register cap for that, the Packed one fits as is.
__global__ __launch_bounds__(kThreads) void packed_decode_kernel(DecodeArgs a) {
  decode_split<true>(a);
}
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) void
native_decode_kernel(DecodeArgs a) {
  decode_split<false>(a);
}

// Merge split partials with the sink. One workgroup (4 waves) per (token,
// head) row: wave w takes splits w, w+4, ...; lane l owns coordinates
// 8l..8l+7; the 4 partial sums meet in LDS in a fixed order.
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ ws_o,
                                                      const float* __restrict__ ws_lse,
                                                      const float* __restrict__ sink, int splits,
                                                      int64_t heads, uint16_t* __restrict__ out,
                                                      float* __restrict__ lse) {
  __shared__ f32x4 part[4][2][64];
  const int lane = wave_lane();
  const int wave = uniform((int)(threadIdx.x >> 6));
  const int64_t row = blockIdx.x;
  const int64_t t = row / heads, h = row - t * heads;
  const float sink2 = sink ? sink[h] * kLog2e : -INFINITY;
  // every wave reads all split LSEs (lane s holds split s; splits <= 64)
  const float ls = lane < splits ? ws_lse[(t * splits + lane) * heads + h] : -INFINITY;
  float mz = fmaxf(ls, sink2);
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) mz = fmaxf(mz, __shfl_xor(mz, d, 64));
  const float w = (mz != -INFINITY && lane < splits) ? exp2f(ls - mz) : 0.0f;
  float z = w;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) z += __shfl_xor(z, d, 64);
  const float* src = ws_o + (t * splits * heads + h) * kHeadDim + 8 * lane;
  const int64_t step = heads * kHeadDim;
  f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
  constexpr int kU = 4;  // splits per batch of in-flight loads, per wave
  for (int s0 = wave; s0 < splits; s0 += 4 * kU) {
    f32x4 x[2 * kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int s = s0 + 4 * u;
      x[2 * u] = s < splits ? *(const f32x4*)(src + s * step) : f32x4{0.f, 0.f, 0.f, 0.f};
      x[2 * u + 1] = s < splits ? *(const f32x4*)(src + s * step + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int s = s0 + 4 * u;
      const float wu = __shfl(w, s < splits ? s : 0, 64);
      const float ww = s < splits ? wu : 0.0f;
      a0 += ww * x[2 * u];
      a1 += ww * x[2 * u + 1];
    }
  }
  part[wave][0][lane] = a0;
  part[wave][1][lane] = a1;
  __syncthreads();
  if (wave == 0) {
    float lse_out = -INFINITY;
    f32x4 r0 = {0.f, 0.f, 0.f, 0.f}, r1 = {0.f, 0.f, 0.f, 0.f};
    if (mz != -INFINITY) {
      const float zt = z + exp2f(sink2 - mz);
      const float inv = 1.0f / zt;
      r0 = (part[0][0][lane] + part[1][0][lane] + part[2][0][lane] + part[3][0][lane]) * inv;
      r1 = (part[0][1][lane] + part[1][1][lane] + part[2][1][lane] + part[3][1][lane]) * inv;
      lse_out = (mz + log2f(zt)) * kLn2;
    }
    *(u32x4*)(out + row * kHeadDim + 8 * lane) =
        u32x4{pack_bf16x2(r0[0], r0[1]), pack_bf16x2(r0[2], r0[3]), pack_bf16x2(r1[0], r1[1]),
              pack_bf16x2(r1[2], r1[3])};
    if (lane == 0) lse[row] = lse_out;
  }
}

struct Plan {
  int splits;
  int chunk;
  size_t bytes;
};

// Aim for one full round of resident workgroups (3 per CU on 256 CUs); a split
// holds whole groups of three tiles, at most kMaxChunk records.
Plan plan_for(int64_t tokens, int64_t heads, int64_t topk) {
  const int64_t base = tokens * (heads / 16);
  const int64_t groups = (topk + 3 * kT - 1) / (3 * kT);  // three-tile groups
  int64_t splits = base > 0 ? (768 + base - 1) / base : 1;
  const int64_t min_splits = (topk + kMaxChunk - 1) / kMaxChunk;
  if (splits > groups) splits = groups;
  if (splits > kMaxSplits) splits = kMaxSplits;
  if (splits < min_splits) splits = min_splits;
  if (splits < 1) splits = 1;
  int64_t chunk_groups = (groups + splits - 1) / splits;
  if (chunk_groups < 1) chunk_groups = 1;
  const int64_t chunk_tiles = 3 * chunk_groups;
  splits = (groups + chunk_groups - 1) / chunk_groups;
  if (splits < 1) splits = 1;
  Plan p;
  p.splits = (int)splits;
  p.chunk = (int)(chunk_tiles * kT);
  p.bytes = splits > 1 ? (size_t)(tokens * splits * heads) * (kHeadDim + 1) * sizeof(float) : 0;
  return p;
}

bool aligned(const void* p, uintptr_t al) { return ((uintptr_t)p & (al - 1)) == 0; }

template <bool kPacked>
int launch_decode(const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads,
                  const uint8_t* pool, int64_t pool_pages, const int32_t* block_table,
                  int64_t bt_stride, int64_t max_blocks, const int32_t* seqlens,
                  const int32_t* indices, int64_t topk, const int32_t* topk_length,
                  const float* sink, const float* freqs, int64_t freq_rows, float scale,
                  uint16_t* out, float* lse, void* workspace, size_t workspace_bytes,
                  void* stream) {
  if (batch < 0 || q_len < 0 || topk < 0 || pool_pages < 0 || max_blocks < 0 || freq_rows < 0)
    return RM_ERR_SHAPE;
  const int64_t tokens = batch * q_len;
  if (tokens == 0 || heads == 0) return RM_OK;
  if (heads < 0 || heads % 16 || heads > 1024 || bt_stride < max_blocks) return RM_ERR_SHAPE;
  if (topk > (int64_t)kMaxChunk * kMaxSplits) return RM_ERR_SHAPE;
  if (pool_pages > ((int64_t)1 << 25)) return RM_ERR_SHAPE;  // slots fit in int32
  if (!q || !out || !lse || (topk > 0 && (!indices || !pool || !block_table)))
    return RM_ERR_NULL;
  if (!aligned(q, 16) || !aligned(out, 16) || (pool && !aligned(pool, 16)) ||
      (freqs && !aligned(freqs, 16)))
    return RM_ERR_ALIGN;
  if (tokens > 65535) return RM_ERR_SHAPE;
  const Plan plan = plan_for(tokens, heads, topk);
  if (plan.bytes > 0 && (!workspace || workspace_bytes < plan.bytes)) return RM_ERR_WORKSPACE;
  if (plan.bytes > 0 && !aligned(workspace, 16)) return RM_ERR_ALIGN;
  DecodeArgs a;
  a.q = q;
  a.pool = pool;
  a.pool_pages = pool_pages;
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
  a.scale_log2 = scale * kLog2e;
  a.q_len = q_len;
  a.heads = heads;
  a.chunk = plan.chunk;
  a.splits = plan.splits;
  a.out = out;
  a.lse = lse;
  a.ws_o = (float*)workspace;
  a.ws_lse = plan.bytes ? (float*)workspace + (size_t)tokens * plan.splits * heads * kHeadDim
                        : nullptr;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(kPacked ? packed_decode_kernel : native_decode_kernel,
                     dim3((unsigned)plan.splits, (unsigned)tokens, (unsigned)(heads / 16)),
                     dim3(kThreads), 0, s, a);
  if (hipGetLastError() != hipSuccess) return RM_ERR_LAUNCH;
  if (plan.splits > 1) {
    const int64_t rows = tokens * heads;
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)rows), dim3(256), 0, s, a.ws_o, a.ws_lse,
                       sink, plan.splits, heads, out, lse);
    if (hipGetLastError() != hipSuccess) return RM_ERR_LAUNCH;
  }
  return RM_OK;
}

}  // namespace

extern "C" int rm_sparse_decode_workspace(int64_t tokens, int64_t heads, int64_t topk,
                                          int32_t* num_splits, size_t* workspace_bytes) {
  if (tokens < 0 || heads < 0 || heads % 16 || topk < 0 ||
      topk > (int64_t)kMaxChunk * kMaxSplits)
    return RM_ERR_SHAPE;
  const Plan p = plan_for(tokens, heads, topk);
  if (num_splits) *num_splits = p.splits;
  if (workspace_bytes) *workspace_bytes = p.bytes;
  return RM_OK;
}

extern "C" int rm_remnant_sparse_decode_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* pool,
    int64_t pool_pages, const int32_t* block_table, int64_t block_table_stride,
    int64_t max_blocks, const int32_t* seqlens, const int32_t* indices, int64_t topk,
    const int32_t* topk_length, const float* sink, const float* freqs, int64_t freq_rows,
    float softmax_scale, uint16_t* out, float* lse, void* workspace, size_t workspace_bytes,
    void* stream) {
  return launch_decode<true>(q, batch, q_len, heads, pool, pool_pages, block_table,
                             block_table_stride, max_blocks, seqlens, indices, topk, topk_length,
                             sink, freqs, freq_rows, softmax_scale, out, lse, workspace,
                             workspace_bytes, stream);
}

extern "C" int rm_native_sparse_decode_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* pool,
    int64_t pool_pages, const int32_t* block_table, int64_t block_table_stride,
    int64_t max_blocks, const int32_t* seqlens, const int32_t* indices, int64_t topk,
    const int32_t* topk_length, const float* sink, float softmax_scale, uint16_t* out,
    float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  return launch_decode<false>(q, batch, q_len, heads, pool, pool_pages, block_table,
                              block_table_stride, max_blocks, seqlens, indices, topk,
                              topk_length, sink, nullptr, 0, softmax_scale, out, lse, workspace,
                              workspace_bytes, stream);
}

extern "C" int rm_version(void) { return 300; }
