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
// Work split. A workgroup of 4 waves owns (split, token, 16-head block) and
// walks its share of the top-k list in tiles of 32 records:
//   * record metadata (index -> block table -> page/row, validity) for the
//     whole share is resolved once into LDS;
//   * the next tile's record bytes (and its RoPE rows) are loaded into
//     registers while the current tile computes, then written to LDS staging;
//   * dequantization: thread (record r, chunk j) expands coordinates
//     64w+8j..64w+8j+7 of every word w -- v_perm places the kept E4M3 codes (zeros for pruned lanes)
//     using a 256-entry selector table, v_cvt_scalef32_pk_bf16_fp8 applies the
//     UE8M0 scale, the tail word is BF16-rounded then rotated -- into a dense
//     BF16 tile K[32][512] in LDS;
//   * QK: wave w contracts its 128-coordinate quarter (S^T = K Q^T on
//     v_mfma_f32_16x16x32_bf16); the 4 partial S^T tiles are summed through LDS;
//   * online softmax in the log2 domain (identical in every wave);
//   * PV: wave w accumulates O[16 heads][its 128 coordinates] on
//     v_mfma_f32_16x16x32_bf16, the P operand taken straight from the S^T
//     accumulator layout and the K operand read with ds_read_b64_tr_b16.
// A split count > 1 writes (O/l, m + log2 l) partials merged with the sink by a
// combine kernel; a single split finalises in place.
#include "remnant_device.h"
#include "remnant_mi355x.h"

using namespace rm;

namespace {

constexpr int kT = 32;                     // records per tile
constexpr int kThreads = 256;              // 4 waves
constexpr int kKdStride = kHeadDim + 8;    // BF16 per LDS row (1040 B, 16-B aligned)
constexpr int kMaxChunk = 1024;            // records per split
constexpr int kMaxSplits = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
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

// Staging geometry. A Packed record (328 B, 8-byte aligned) is fetched as the 21
// aligned 16-byte pieces covering it -- an even row's last piece reaches 8 bytes
// into the next row of the same page, which always exists because row 63 is odd
// -- and written to its 336-byte staging row shifted so the record starts at 0. A Native record stages
// its 576-byte data row (36 pieces) plus its 8-byte scale row.
template <bool kPacked>
struct Geo {
  static constexpr int kData = kPacked ? kRecordBytes : kNativeDataBytes;  // row pitch
  static constexpr int kPage = kPacked ? kPageBytes : kNativePageBytes;
  static constexpr int kPieces = kPacked ? 21 : kNativeDataBytes / 16;
  static constexpr int kStage = kPacked ? 336 : kNativeDataBytes + 16;
  static constexpr int kDataChunks = kT * kPieces;      // 16-byte pieces per tile
  static constexpr int kDataLoads = (kDataChunks + kThreads - 1) / kThreads;
  static constexpr int kFreqLoads = kPacked ? (kT * 256 / 16) / kThreads : 0;  // 2
};

template <bool kPacked>
struct Smem {
  uint16_t kd[kT * kKdStride];                       // dense BF16 tile
  uint8_t stage[kT * Geo<kPacked>::kStage];          // raw records of the tile
  float freq[kPacked ? kT * 64 : 1];                 // RoPE rows of the tile
  f32x4 spart[4][2][64];                             // per-wave partial S^T
  uint64_t sel[kPacked ? 256 : 1];                   // v_perm selectors per bitmap byte
  int32_t rec[kMaxChunk];                            // slot (page*64+row) or -1
  int32_t raw[kMaxChunk];
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

template <bool kPacked>
__global__ __launch_bounds__(kThreads, 2) void sparse_decode_kernel(DecodeArgs a) {
  using G = Geo<kPacked>;
  __shared__ __attribute__((aligned(16))) Smem<kPacked> sm;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
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

  // ---- setup: selectors, record metadata, Q operand ----
  if (kPacked) {
    // byte bits MSB-first = coordinates 0..7; selector byte i = rank of i or 0x0c (zero)
    uint32_t s = tid, r = 0;
    uint64_t sel = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool kept = (s >> (7 - i)) & 1u;
      sel |= (uint64_t)(kept ? r : 0x0cu) << (8 * i);
      r += kept ? 1u : 0u;
    }
    sm.sel[tid] = sel;
  }
  for (int i = tid; i < n; i += kThreads) {
    const int64_t r = a.indices[t * a.topk + k0 + i];
    bool ok = r >= 0 && r < seqlen && (r >> 6) < a.max_blocks;
    int64_t page = ok ? a.block_table[b * a.bt_stride + (r >> 6)] : -1;
    ok = ok && page >= 0 && page < a.pool_pages;
    if (kPacked && a.freqs) ok = ok && r * 4 < a.freq_rows;
    sm.rec[i] = ok ? (int32_t)(page * 64 + (r & 63)) : -1;
    sm.raw[i] = (int32_t)r;
  }
  bf16x8 qreg[4];  // Q[head col][128 wave + 32 ks + 8 g .. +7]
  {
    const uint16_t* qh = a.q + (t * a.heads + head0 + col) * kHeadDim + 128 * wave + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qreg[ks] = __builtin_bit_cast(bf16x8, *(const u32x4*)(qh + 32 * ks));
  }
  f32x4 o[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  __syncthreads();

  // ---- tile loader: registers <- HBM, LDS staging <- registers ----
  u32x4 pre[G::kDataLoads];
  u32x2 pre_scale;
  u32x4 pre_freq[G::kFreqLoads > 0 ? G::kFreqLoads : 1];
  int base_next = 0;  // first record of the tile held in the prefetch registers
  auto load_tile = [&](int base) {
    base_next = base;
#pragma unroll
    for (int j = 0; j < G::kDataLoads; ++j) {
      const int c = tid + j * kThreads;
      pre[j] = u32x4{0u, 0u, 0u, 0u};
      // the bound is wave-uniform (whole waves drop out of the last round)
      if (c < G::kDataChunks) {
        const int r = c / G::kPieces, piece = c % G::kPieces;
        const int slot = base + r < n ? sm.rec[base + r] : -1;
        if (slot >= 0) {
          const uint8_t* row = a.pool + (int64_t)(slot >> 6) * G::kPage + (slot & 63) * G::kData;
          // Packed: odd rows start 8 bytes past a 16-byte boundary and are fetched
          // from 8 bytes earlier; an even row's last piece runs 8 bytes into the
          // next row of the same page (row 63, the last, is odd): always in bounds
          pre[j] = *(const u32x4*)(row - (kPacked ? 8 * (slot & 1) : 0) + 16 * piece);
        }
      }
    }
    if (!kPacked) {
      pre_scale = u32x2{0u, 0u};
      if (tid < kT) {
        const int slot = base + tid < n ? sm.rec[base + tid] : -1;
        if (slot >= 0) {
          const uint8_t* page = a.pool + (int64_t)(slot >> 6) * G::kPage;
          pre_scale = *(const u32x2*)(page + kPageRecords * G::kData + (slot & 63) * kScaleBytes);
        }
      }
    }
    if (kPacked) {
#pragma unroll
      for (int j = 0; j < G::kFreqLoads; ++j) {
        const int c = tid + j * kThreads;  // 16 pieces of 16 B per record
        const int r = c >> 4, piece = c & 15;
        const int slot = base + r < n ? sm.rec[base + r] : -1;
        pre_freq[j] = u32x4{0u, 0u, 0u, 0u};
        if (slot >= 0 && a.freqs) {
          const int64_t raw = sm.raw[base + r];
          pre_freq[j] = *(const u32x4*)(a.freqs + raw * 4 * 64 + 4 * piece);
        }
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < G::kDataLoads; ++j) {
      const int c = tid + j * kThreads;
      if (c < G::kDataChunks) {
        const int r = c / G::kPieces, piece = c % G::kPieces;
        uint8_t* st = sm.stage + r * G::kStage;
        if (kPacked) {
          // odd pool rows were fetched from 8 bytes before the record: shift them
          // down so every staged record starts at offset 0 (the first half-piece
          // of an odd row lands in the row's unused pad bytes 328..335)
          const int rs = base_next + r < n ? sm.rec[base_next + r] : 0;
          const int odd = rs & 1;
          const int lo_at = odd ? (piece ? 16 * piece - 8 : kRecordBytes) : 16 * piece;
          const int hi_at = 16 * piece + (odd ? 0 : 8);
          *(u32x2*)(st + lo_at) = u32x2{pre[j][0], pre[j][1]};
          *(u32x2*)(st + hi_at) = u32x2{pre[j][2], pre[j][3]};
        } else {
          *(u32x4*)(st + 16 * piece) = pre[j];
        }
      }
    }
    if (!kPacked && tid < kT) *(u32x2*)(sm.stage + tid * G::kStage + G::kData) = pre_scale;
    if (kPacked) {
#pragma unroll
      for (int j = 0; j < G::kFreqLoads; ++j) {
        const int c = tid + j * kThreads;
        *(u32x4*)(sm.freq + (c >> 4) * 64 + 4 * (c & 15)) = pre_freq[j];
      }
    }
  };

  // prologue: tile 0 staged, tile 1 in flight
  if (n > 0) {
    load_tile(0);
    store_tile();
  }
  __syncthreads();
  if (kT < n) load_tile(kT);

  for (int base = 0; base < n; base += kT) {

    // ---- dequantize: thread (record r = tid/8, chunk j = tid%8) expands chunk j of
    // every 64-coordinate word; the RoPE tail (word 7) is one unrolled iteration,
    // uniform across the wave ----
    {
      const int r = tid >> 3, j = tid & 7;
      const uint8_t* st = sm.stage + r * G::kStage;
      uint16_t* krow = sm.kd + r * kKdStride + 8 * j;
      if (kPacked) {
        uint64_t wd[8];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          const u32x2 v = *(const u32x2*)(st + kCodeBytes + 8 * w);
          wd[w] = ((uint64_t)v[1] << 32) | v[0];
        }
        const u32x2 sb = *(const u32x2*)(st + kDataBytes);
        const uint64_t before = ~(~0ull >> (8 * j));  // coordinates of earlier chunks in a word
        int base_rank = 0;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          const uint32_t byte = (uint32_t)(wd[w] >> (56 - 8 * j)) & 0xffu;
          const int rank = base_rank + __popcll(wd[w] & before);
          base_rank += __popcll(wd[w]);
          const uint32_t* cw = (const uint32_t*)(st + (rank & ~3));
          const uint32_t d0 = cw[0], d1 = cw[1], d2 = cw[2];
          const uint32_t lo4 = __builtin_amdgcn_alignbyte(d1, d0, (uint32_t)rank & 3u);
          const uint32_t hi4 = __builtin_amdgcn_alignbyte(d2, d1, (uint32_t)rank & 3u);
          const uint64_t sel = sm.sel[byte];
          const uint32_t lo = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)sel);
          const uint32_t hi = __builtin_amdgcn_perm(hi4, lo4, (uint32_t)(sel >> 32));
          const float scale = exp2i((int)((sb[w >> 2] >> (8 * (w & 3))) & 0xffu) - 127);
          u32x4 v = {cvt2<false>(lo, scale), cvt2<true>(lo, scale), cvt2<false>(hi, scale),
                     cvt2<true>(hi, scale)};
          if (w == 7 && a.freqs) {  // tail: rotate BF16 pairs with the record's RoPE row
            const f32x4 f0 = *(const f32x4*)(sm.freq + r * 64 + 8 * j);
            const f32x4 f1 = *(const f32x4*)(sm.freq + r * 64 + 8 * j + 4);
            float x[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              x[2 * i] = u2f(v[i] << 16);
              x[2 * i + 1] = u2f(v[i] & 0xffff0000u);
            }
            float cs[8] = {f0[0], f0[1], f0[2], f0[3], f1[0], f1[1], f1[2], f1[3]};
            rope4(x, cs);
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
          }
          *(u32x4*)(krow + 64 * w) = v;
        }
      } else {
        // Native: thread (r, j) converts chunk j of each NoPE word and copies
        // tail chunk j, so every lane runs the same path
        uint16_t* nrow = krow;
        const u32x2 sb = *(const u32x2*)(st + kNativeDataBytes);
#pragma unroll
        for (int ww = 0; ww < 8; ++ww) {
          u32x4 v;
          if (ww < 7) {
            const float scale = exp2i((int)((sb[ww >> 2] >> (8 * (ww & 3))) & 0xffu) - 127);
            const u32x2 codes = *(const u32x2*)(st + 64 * ww + 8 * j);
            v = u32x4{cvt2<false>(codes[0], scale), cvt2<true>(codes[0], scale),
                      cvt2<false>(codes[1], scale), cvt2<true>(codes[1], scale)};
          } else {
            v = *(const u32x4*)(st + kNopeDim + 16 * j);
          }
          *(u32x4*)(nrow + 64 * ww) = v;
        }
      }
    }
    __syncthreads();  // K tile ready; staging free

    // validity of the tile's records as a bit mask (records >= n are invalid)
    const int my = base + (lane & 31);
    const uint32_t vmask =
        (uint32_t)__ballot((lane < 32) && my < n && sm.rec[my < n ? my : 0] >= 0);

    // ---- QK partial over this wave's coordinate quarter ----
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 kv = __builtin_bit_cast(
            bf16x8, *(const u32x4*)(sm.kd + (16 * rb + col) * kKdStride + 128 * wave + 32 * ks + 8 * g));
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qreg[ks], s, 0, 0, 0);
      }
      sm.spart[wave][rb][lane] = s;
    }
    __syncthreads();  // partial S ready

    // ---- online softmax: lane holds records {rb*16 + 4g + i} for head col ----
    float sv[8];
    float mt = -INFINITY;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const f32x4 s = sm.spart[0][rb][lane] + sm.spart[1][rb][lane] + sm.spart[2][rb][lane] +
                      sm.spart[3][rb][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool v = (vmask >> (16 * rb + 4 * g + i)) & 1u;
        sv[4 * rb + i] = v ? s[i] * a.scale_log2 : -INFINITY;
        mt = fmaxf(mt, sv[4 * rb + i]);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = m_new == -INFINITY ? 1.0f : exp2f(m_run - m_new);
    float p[8], psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = m_new == -INFINITY ? 0.0f : exp2f(sv[i] - m_new);
      psum += p[i];
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    if (__ballot(alpha != 1.0f)) {  // some head's running max moved: rescale O
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ai = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) o[nt][i] *= ai;
      }
    }

    // ---- PV: O[head][coord] += P[head][rec] K[rec][coord] ----
    const bf16x8 pab = {(__bf16)p[0], (__bf16)p[1], (__bf16)p[2], (__bf16)p[3],
                        (__bf16)p[4], (__bf16)p[5], (__bf16)p[6], (__bf16)p[7]};
    {
      // lane (g, j) points at K[4g + j/4 (+16)][coord base + 4(j%4)]; receives
      // K[4g + 0..3 (+16)][coord base + j] (transpose read)
      const int j = col;
      const uint16_t* r0 = sm.kd + (4 * g + (j >> 2)) * kKdStride + 128 * wave + 4 * (j & 3);
      const uint16_t* r1 = r0 + 16 * kKdStride;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const s16x4 b0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(r0 + 16 * nt));
        const s16x4 b1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(r1 + 16 * nt));
        const s16x8 bb = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        o[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pab, __builtin_bit_cast(bf16x8, bb), o[nt],
                                                        0, 0, 0);
      }
    }
    // the next tile's bytes were requested one iteration ago: stage them, then
    // request the tile after it so its latency overlaps a whole iteration
    if (base + kT < n) store_tile();
    if (base + 2 * kT < n) load_tile(base + 2 * kT);
    __syncthreads();  // K tile consumed; next tile staged
  }
  // lane holds O[head 4g + i][coord 128 wave + 16 nt + col]; softmax state of head col

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
    if (wave == 0 && lane < 16) a.lse[t * a.heads + head0 + col] = lse;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = __shfl(factor, 4 * g + i, 64);
      uint16_t* orow = a.out + (t * a.heads + head0 + 4 * g + i) * kHeadDim + 128 * wave + col;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) orow[16 * nt] = (uint16_t)bf16_rne(o[nt][i] * f);
    }
  } else {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const float plse = l_run > 0.0f ? m_run + log2f(l_run) : -INFINITY;
    const int64_t slot = (t * a.splits + split) * a.heads + head0;
    if (wave == 0 && lane < 16) a.ws_lse[slot + col] = plse;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = __shfl(inv, 4 * g + i, 64);
      float* orow = a.ws_o + (slot + 4 * g + i) * kHeadDim + 128 * wave + col;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) orow[16 * nt] = o[nt][i] * f;
    }
  }
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

// Aim for ~2 workgroups per CU (256 CUs); each split holds <= kMaxChunk records.
Plan plan_for(int64_t tokens, int64_t heads, int64_t topk) {
  const int64_t base = tokens * (heads / 16);
  const int64_t tiles = (topk + kT - 1) / kT;
  int64_t splits = base > 0 ? (512 + base - 1) / base : 1;
  const int64_t min_splits = (topk + kMaxChunk - 1) / kMaxChunk;
  if (splits > tiles) splits = tiles;
  if (splits > kMaxSplits) splits = kMaxSplits;
  if (splits < min_splits) splits = min_splits;
  if (splits < 1) splits = 1;
  int64_t chunk_tiles = (tiles + splits - 1) / splits;
  if (chunk_tiles < 1) chunk_tiles = 1;
  splits = (tiles + chunk_tiles - 1) / chunk_tiles;
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
  hipLaunchKernelGGL(sparse_decode_kernel<kPacked>,
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

extern "C" int rm_version(void) { return 200; }
