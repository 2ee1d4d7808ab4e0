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
// Work split: one wave64 per (split, token, 16-head block). A split walks its
// share of the top-k list in tiles of 16 records:
//   1. gather: record r -> page block_table[b, r/64], row r%64;
//   2. dequantize the tile (with tail RoPE for Packed) into an LDS tile
//      K[16][512] BF16 -- lanes 4r..4r+3 each expand 128 coordinates of record r;
//   3. S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (Q held in registers);
//   4. online softmax in the log2 domain (one head per lane column);
//   5. O += P K on v_mfma_f32_16x16x16_bf16 (P taken straight from the S^T
//      accumulator layout, K read from the LDS tile).
// Splits write (O/l, log2 l + m) partials that a combine kernel merges with
// the sink; a single split finalises in place.
#include "remnant_device.h"
#include "remnant_mi355x.h"

using namespace rm;

namespace {

constexpr int kTile = 16;
constexpr int kKdStride = kHeadDim + 8;  // BF16 elements per LDS row (pad vs bank conflicts)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef short s16x4 __attribute__((ext_vector_type(4)));

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
  int chunk;       // records per split (multiple of kTile)
  int splits;
  uint16_t* out;
  float* lse;
  float* ws_o;     // [tokens, splits, heads, 512]
  float* ws_lse;   // [tokens, splits, heads]
};

// Expand 8 coordinates of a Packed record (bitmap byte MSB-first, kept codes
// as the next bytes of `run`) to BF16-rounded floats.
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

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return bf16_rne(a) | (bf16_rne(b) << 16);
}

// Lane (record rec, quarter qt) writes coordinates 128qt..128qt+127 of its record.
template <bool kPacked>
__device__ __forceinline__ void dequant_quarter(const DecodeArgs& a, const uint8_t* rec_data,
                                                const uint8_t* rec_scales, int64_t raw, bool ok,
                                                int qt, uint16_t* kd_row) {
  if (!ok) {
#pragma unroll 4
    for (int c = 0; c < 16; ++c) *(u32x4*)(kd_row + 128 * qt + 8 * c) = u32x4{0u, 0u, 0u, 0u};
    return;
  }
  if (kPacked) {
    const u32x4* bm = (const u32x4*)(rec_data + kCodeBytes);
    const u32x4 b0 = bm[0], b1 = bm[1], b2 = bm[2], b3 = bm[3];
    const uint64_t w[8] = {((uint64_t)b0[1] << 32) | b0[0], ((uint64_t)b0[3] << 32) | b0[2],
                           ((uint64_t)b1[1] << 32) | b1[0], ((uint64_t)b1[3] << 32) | b1[2],
                           ((uint64_t)b2[1] << 32) | b2[0], ((uint64_t)b2[3] << 32) | b2[2],
                           ((uint64_t)b3[1] << 32) | b3[0], ((uint64_t)b3[3] << 32) | b3[2]};
    int rank = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) rank += i < 2 * qt ? __popcll(w[i]) : 0;
    const uint64_t wa = qt == 0 ? w[0] : qt == 1 ? w[2] : qt == 2 ? w[4] : w[6];
    const uint64_t wb = qt == 0 ? w[1] : qt == 1 ? w[3] : qt == 2 ? w[5] : w[7];
    const float sa = exp2i((int)rec_scales[2 * qt] - 127);
    const float sb = exp2i((int)rec_scales[2 * qt + 1] - 127);
    const float* fr = a.freqs ? a.freqs + (raw * 4) * (2 * kRopePairs) : nullptr;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const uint64_t word = c < 8 ? wa : wb;
      const uint32_t bits = (uint32_t)(word >> (56 - 8 * (c & 7))) & 0xffu;
      const int base = rank & ~3;
      const uint32_t* cw = (const uint32_t*)(rec_data + base);
      const uint32_t d0 = cw[0], d1 = cw[1], d2 = cw[2];
      const uint32_t sh = 8u * (uint32_t)(rank & 3);
      const uint32_t lo = (uint32_t)((((uint64_t)d1 << 32) | d0) >> sh);
      const uint32_t hi = (uint32_t)((((uint64_t)d2 << 32) | d1) >> sh);
      float v[8];
      expand8(bits, ((uint64_t)hi << 32) | lo, c < 8 ? sa : sb, v);
      rank += __popc(bits);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = bf16_to_f32(bf16_rne(v[i]));
      const int coord = 128 * qt + 8 * c;
      if (qt == 3 && c >= 8 && fr) {  // coordinates 448..511: rotate in place
        // coordinate 448 + 2j is the real part of pair j: (cos, sin) at floats 2j, 2j + 1
        const float* f = fr + (coord - kNopeDim);
        const f32x4 x0 = *(const f32x4*)f, x1 = *(const f32x4*)(f + 4);
        float cs[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        rope4(v, cs);
      }
      *(u32x4*)(kd_row + coord) = u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                        pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
    }
  } else {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int coord = 128 * qt + 8 * c;
      if (coord < kNopeDim) {
        const u32x2 codes = *(const u32x2*)(rec_data + coord);
        const float s = exp2i((int)rec_scales[coord / kGroup] - 127);
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = e4m3_to_f32((codes[0] >> (8 * i)) & 0xffu) * s;
          v[4 + i] = e4m3_to_f32((codes[1] >> (8 * i)) & 0xffu) * s;
        }
        *(u32x4*)(kd_row + coord) = u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                          pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
      } else {
        *(u32x4*)(kd_row + coord) = *(const u32x4*)(rec_data + kNopeDim + 2 * (coord - kNopeDim));
      }
    }
  }
}

template <bool kPacked>
__global__ __launch_bounds__(64) void sparse_decode_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t kd[kTile * kKdStride];
  const int lane = wave_lane();
  const int split = blockIdx.x;
  const int64_t t = blockIdx.y;
  const int hb = blockIdx.z;
  const int64_t b = t / a.q_len;
  const int g = lane >> 4, col = lane & 15;
  const int64_t head0 = (int64_t)hb * 16;

  int64_t len = a.topk;
  if (a.topk_length) {
    const int64_t l = a.topk_length[t];
    len = l < 0 ? 0 : (l < a.topk ? l : a.topk);
  }
  const int64_t k0 = (int64_t)split * a.chunk;
  const int64_t k1 = k0 + a.chunk < len ? k0 + a.chunk : len;
  const int64_t seqlen = a.seqlens ? a.seqlens[b] : INT64_MAX;
  const int64_t pool_bytes_page = kPacked ? kPageBytes : kNativePageBytes;
  const int data_bytes = kPacked ? kDataBytes : kNativeDataBytes;

  // Q^T operand: lane (col = head, g) holds Q[head][32ks + 8g .. +7]
  bf16x8 qreg[16];
  {
    const uint16_t* qh = a.q + ((t * a.heads) + head0 + col) * kHeadDim + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) qreg[ks] = __builtin_bit_cast(bf16x8, *(const u32x4*)(qh + 32 * ks));
  }
  f32x4 o[32];
#pragma unroll
  for (int nt = 0; nt < 32; ++nt) o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;  // softmax state of head `col`

  for (int64_t kt = k0; kt < k1; kt += kTile) {
    // 1. gather metadata: lanes 0..15 resolve records kt..kt+15
    const int64_t k = kt + (lane & 15);
    bool ok = lane < kTile && k < k1;
    int64_t r = ok ? a.indices[t * a.topk + k] : -1;
    ok = ok && r >= 0 && r < seqlen && (r >> 6) < a.max_blocks;
    int64_t page = ok ? a.block_table[b * a.bt_stride + (r >> 6)] : -1;
    ok = ok && page >= 0 && page < a.pool_pages;
    if (kPacked && a.freqs) ok = ok && r * 4 < a.freq_rows;
    const uint32_t vmask = (uint32_t)__ballot(ok);

    // 2. dequantize: lane -> record lane/4, quarter lane%4
    {
      const int rec = lane >> 2, qt = lane & 3;
      const int64_t rr = __shfl(r, rec, 64);
      const int64_t pg = __shfl(page, rec, 64);
      const bool rok = (vmask >> rec) & 1u;
      const uint8_t* base = a.pool + (rok ? pg : 0) * pool_bytes_page;
      const int row = (int)(rr & 63);
      dequant_quarter<kPacked>(a, base + row * data_bytes,
                               base + kPageRecords * data_bytes + row * kScaleBytes, rr, rok, qt,
                               kd + rec * kKdStride);
    }
    wave_lds_sync();

    // 3. S^T[rec][head] = K[rec] . Q[head]
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      const bf16x8 kv = __builtin_bit_cast(bf16x8, *(const u32x4*)(kd + col * kKdStride + 32 * ks + 8 * g));
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qreg[ks], s, 0, 0, 0);
    }
    // lane holds S^T[rec = 4g + i][head = col]

    // 4. online softmax (log2 domain)
    float sv[4];
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool v = (vmask >> (4 * g + i)) & 1u;
      sv[i] = v ? s[i] * a.scale_log2 : -INFINITY;
      mt = fmaxf(mt, sv[i]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = m_new == -INFINITY ? 1.0f : exp2f(m_run - m_new);
    float p[4], psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = m_new == -INFINITY ? 0.0f : exp2f(sv[i] - m_new);
      psum += p[i];
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // rescale O rows (heads 4g + i) by their heads' alpha
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ai = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
      for (int nt = 0; nt < 32; ++nt) o[nt][i] *= ai;
    }

    // 5. O[head][coord] += P[head][rec] K[rec][coord]; P operand = S^T layout
    s16x4 pa;
#pragma unroll
    for (int i = 0; i < 4; ++i) pa[i] = (short)bf16_rne(p[i]);
#pragma unroll
    for (int nt = 0; nt < 32; ++nt) {
      s16x4 kb;
#pragma unroll
      for (int j = 0; j < 4; ++j) kb[j] = (short)kd[(4 * g + j) * kKdStride + 16 * nt + col];
      o[nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, kb, o[nt], 0, 0, 0);
    }
    wave_lds_sync();
  }
  // lane holds O[head 4g + i][coord 16nt + col]; softmax state of head col

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
    if (lane < 16) a.lse[t * a.heads + head0 + col] = lse;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = __shfl(factor, 4 * g + i, 64);
      uint16_t* orow = a.out + (t * a.heads + head0 + 4 * g + i) * kHeadDim + col;
#pragma unroll
      for (int nt = 0; nt < 32; ++nt) orow[16 * nt] = (uint16_t)bf16_rne(o[nt][i] * f);
    }
  } else {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const float plse = l_run > 0.0f ? m_run + log2f(l_run) : -INFINITY;
    const int64_t slot = (t * a.splits + split) * a.heads + head0;
    if (lane < 16) a.ws_lse[slot + col] = plse;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = __shfl(inv, 4 * g + i, 64);
      float* orow = a.ws_o + (slot + 4 * g + i) * kHeadDim + col;
#pragma unroll
      for (int nt = 0; nt < 32; ++nt) orow[16 * nt] = o[nt][i] * f;
    }
  }
}

// Merge split partials with the sink: one wave per (token, head), 8 coords/lane.
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ ws_o,
                                                      const float* __restrict__ ws_lse,
                                                      const float* __restrict__ sink, int splits,
                                                      int64_t heads, int64_t rows,
                                                      uint16_t* __restrict__ out,
                                                      float* __restrict__ lse) {
  const int lane = wave_lane();
  const int64_t row = (int64_t)blockIdx.x * 4 + uniform((int)(threadIdx.x >> 6));
  if (row >= rows) return;
  const int64_t t = row / heads, h = row - t * heads;
  const float sink2 = sink ? sink[h] * kLog2e : -INFINITY;
  float mz = sink2;
  for (int s = 0; s < splits; ++s) mz = fmaxf(mz, ws_lse[(t * splits + s) * heads + h]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float lse_out = -INFINITY;
  if (mz != -INFINITY) {
    float z = exp2f(sink2 - mz);
    for (int s = 0; s < splits; ++s) {
      const int64_t slot = (t * splits + s) * heads + h;
      const float w = exp2f(ws_lse[slot] - mz);
      z += w;
      if (w > 0.0f) {
        const float* src = ws_o + slot * kHeadDim + 8 * lane;
        const f32x4 x0 = *(const f32x4*)src, x1 = *(const f32x4*)(src + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i] += w * x0[i];
          acc[4 + i] += w * x1[i];
        }
      }
    }
    const float inv = 1.0f / z;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= inv;
    lse_out = (mz + log2f(z)) * kLn2;
  }
  *(u32x4*)(out + row * kHeadDim + 8 * lane) =
      u32x4{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]), pack_bf16x2(acc[4], acc[5]),
            pack_bf16x2(acc[6], acc[7])};
  if (lane == 0) lse[row] = lse_out;
}

struct Plan {
  int splits;
  int chunk;
  size_t bytes;
};

Plan plan_for(int64_t tokens, int64_t heads, int64_t topk) {
  const int64_t base = tokens * (heads / 16);
  const int64_t max_splits = (topk + kTile - 1) / kTile;
  int64_t splits = base > 0 ? (512 + base - 1) / base : 1;
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  int64_t chunk = (topk + splits - 1) / splits;
  chunk = (chunk + kTile - 1) / kTile * kTile;
  if (chunk < kTile) chunk = kTile;
  splits = (topk + chunk - 1) / chunk;
  if (splits < 1) splits = 1;
  Plan p;
  p.splits = (int)splits;
  p.chunk = (int)chunk;
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
                     dim3(64), 0, s, a);
  if (hipGetLastError() != hipSuccess) return RM_ERR_LAUNCH;
  if (plan.splits > 1) {
    const int64_t rows = tokens * heads;
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s,
                       a.ws_o, a.ws_lse, sink, plan.splits, heads, rows, out, lse);
    if (hipGetLastError() != hipSuccess) return RM_ERR_LAUNCH;
  }
  return RM_OK;
}

}  // namespace

extern "C" int rm_sparse_decode_workspace(int64_t tokens, int64_t heads, int64_t topk,
                                          int32_t* num_splits, size_t* workspace_bytes) {
  if (tokens < 0 || heads < 0 || heads % 16 || topk < 0) return RM_ERR_SHAPE;
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

extern "C" int rm_version(void) { return 100; }
