/*
 * remnant_mi355x.h -- C ABI of the MI355X (gfx950) Remnant packed-KV hot path.
 *
 * Plain pointers and sizes only: device pointers for tensors, a hipStream_t
 * passed as void*. Every entry point is asynchronous on the given stream,
 * allocates nothing, and returns an rm_status (0 = ok, negative = rejected
 * argument; nothing was launched). Empty inputs return RM_OK without a launch.
 *
 * Pool geometry (identical for every entry point):
 *   Packed page (20,992 B) = 64 contiguous 328-byte records: 256 E4M3 codes in
 *   ascending coordinate order, then 8 little-endian uint64 bitmap words
 *   (MSB-first: coordinate c is bit 63 - c % 64 of word c / 64), then 8 UE8M0
 *   scale bytes (one per 64-coordinate group). Records are 8-byte aligned.
 *   Native page (37,376 B) = 64 data rows of 576 B (448 E4M3 codes, 64 rotated
 *   BF16) followed by 64 scale rows (7 UE8M0 bytes + 1 zero byte). 584 B/record.
 *   Pool slot s lives in page s / 64, row s % 64.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   rm_pack_rows              fork srt/remnant/packed.py::pack_rows_fused and the
 *                             fused Triton store (third_party/README.md:257,
 *                             378-381; called from compressor_v2.py store dispatch)
 *   rm_native_store_rows      stock fused_norm_rope_flashmla store (Native control;
 *                             decode-store manifest.json source.native_store)
 *   rm_unpack_gather_bf16     srt/remnant/packed.py::unpack_gather_bf16
 *                             (benchmarks/microbench/dsv4-flash-prefill-read-fused-rope/
 *                             candidate-sglang.patch:427-480, kernels :502-668)
 *   rm_remnant_sparse_decode_fwd
 *                             sgl_kernel/flash_mla.py::remnant_sparse_decode_fwd,
 *                             FlashMLA csrc/api/sparse_decode.h Direct decode +
 *                             combine (third_party/README.md:260, 351-361;
 *                             Dockerfile.v0.5.18:56-57)
 *   rm_native_sparse_decode_fwd
 *                             stock FlashMLA sparse FP8 decode on 584-B records
 *                             (Native control, same harness)
 *   rm_sparse_decode_workspace  FlashMLA get_mla_metadata-style split planning
 *   rm_remnant_sparse_decode_swa_fwd / rm_native_sparse_decode_swa_fwd /
 *   rm_sparse_decode_workspace_swa
 *                             the same decodes attending the sliding-window (SWA)
 *                             rows jointly with the C4 top-k and the sink, as the
 *                             reference decode does (decode-store timing.json
 *                             swa_length 64; joint softmax training/losses.py:393-398)
 *   rm_packed_to_native       the CUDA Adapter (SGLang csrc/remnant/packed_to_native.cu,
 *                             third_party/README.md:259, 289) and the Triton
 *                             _bf16_to_native_kernel step of the Triton decode
 *   rm_copy_records           the host-cache (HiCache) coordinated value/bitmap/scale
 *                             transfers (srt/mem_cache/memory_pool_host.py,
 *                             third_party/README.md:261)
 *   rm_pack_rows_k / rm_unpack_gather_bf16_k
 *                             the survivor-profile store and reader
 *                             (configure_cache_format(..., keep_count=K) with the
 *                             KEEP_K Triton kernels: candidate-sglang.patch:471-479,
 *                             707-736, 775-790; docs/agents/numerical-and-validation.md:10-14)
 *   rm_pack_rows_planes / rm_unpack_gather_bf16_planes / rm_packed_to_native_planes /
 *   rm_remnant_sparse_decode_planes_fwd
 *                             the same operators on the reference's plane-form pool
 *                             buffers (values, bitmaps, scales): packed.py::_as_buffers
 *                             and the callers passing the plane tuple
 *                             (candidate-sglang.patch:782-789, 839, 900-911); the decode
 *                             side of sgl_kernel/flash_mla.py::remnant_buffers
 *                             (Dockerfile.v0.5.18:56)
 *
 * Survivor profiles: a Packed pool may instead hold records with K survivors,
 * K = 64..448 in steps of 64: K E4M3 codes, the same 64 bitmap bytes and 8 scale
 * bytes (K + 72 bytes, 8-byte aligned), 64 records per page (64 * (K + 72) B).
 * The sparse decode reads the 256-survivor format only.
 *
 * Plane form: the same records held as three row-aligned planes, slot s being
 * row s of each: values [rows, K] u8 (codes, ascending coordinate), bitmaps
 * [rows, 8] u64 (the bitmap words as above) and scales [rows, 8] u8. Byte for
 * byte the record is values row + bitmaps row + scales row.
 */
#ifndef REMNANT_MI355X_H
#define REMNANT_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum rm_status {
  RM_OK = 0,
  RM_ERR_NULL = -1,      /* required pointer missing */
  RM_ERR_SHAPE = -2,     /* size/stride out of range */
  RM_ERR_ALIGN = -3,     /* pointer not aligned as documented */
  RM_ERR_DTYPE = -4,     /* unsupported dtype code */
  RM_ERR_WORKSPACE = -5, /* workspace too small */
  RM_ERR_LAUNCH = -6     /* the HIP runtime rejected the launch */
};

enum rm_dtype { RM_F32 = 0, RM_BF16 = 1 };

enum rm_format { RM_FORMAT_PACKED = 0, RM_FORMAT_NATIVE = 1 };

#define RM_HEAD_DIM 512
#define RM_NOPE_DIM 448
#define RM_ROPE_PAIRS 32
#define RM_KEEP_COUNT 256
#define RM_PAGE_RECORDS 64
#define RM_PACKED_DATA_BYTES 320
#define RM_PACKED_RECORD_BYTES 328
#define RM_PACKED_PAGE_BYTES 20992
#define RM_NATIVE_DATA_BYTES 576
#define RM_NATIVE_RECORD_BYTES 584
#define RM_NATIVE_PAGE_BYTES 37376

/* Library version (major * 10000 + minor * 100 + patch). */
int rm_version(void);

/* Store: pack n latent rows into Packed records.
 * x: [n, 512] with row stride x_row_stride elements, dtype RM_F32 or RM_BF16
 *    (raw compressor output; 16-byte aligned rows).
 * weight: [512] f32 RMSNorm weight. eps: RMSNorm epsilon.
 * dst_slot: [n] int32 pool slots; a slot < 0 or >= pool_pages * 64 is skipped.
 * pool: packed pages (16-byte aligned). */
int rm_pack_rows(const void* x, int x_dtype, int64_t x_row_stride, const float* weight,
                 float eps, const int32_t* dst_slot, int64_t n, uint8_t* pool,
                 int64_t pool_pages, void* stream);

/* rm_pack_rows for a pool of keep_count-survivor records (keep_count 64..448,
 * a multiple of 64; other values give RM_ERR_SHAPE). rm_pack_rows is this
 * entry point with keep_count 256. */
int rm_pack_rows_k(const void* x, int x_dtype, int64_t x_row_stride, const float* weight,
                   float eps, const int32_t* dst_slot, int64_t n, uint8_t* pool,
                   int64_t pool_pages, int keep_count, void* stream);

/* rm_pack_rows_k writing plane-form buffers: record dst_slot[i] goes to row
 * dst_slot[i] of each plane (a slot < 0 or >= rows is skipped). Planes 8-byte
 * aligned. */
int rm_pack_rows_planes(const void* x, int x_dtype, int64_t x_row_stride, const float* weight,
                        float eps, const int32_t* dst_slot, int64_t n, uint8_t* values,
                        uint64_t* bitmaps, uint8_t* scales, int64_t rows, int keep_count,
                        void* stream);

/* Native control store: unpruned RMSNorm, 7 NoPE groups as UE8M0/E4M3, tail
 * rotated with freqs row position[i] * 4 (freqs: [freq_rows, 32] complex64 as
 * interleaved f32 (cos, sin); NULL = no rotation). Rows whose slot is out of
 * range, or (with freqs) whose position * 4 is outside [0, freq_rows), are skipped. */
int rm_native_store_rows(const void* x, int x_dtype, int64_t x_row_stride,
                         const float* weight, float eps, const int32_t* dst_slot,
                         const int32_t* position, const float* freqs, int64_t freq_rows,
                         int64_t n, uint8_t* pool, int64_t pool_pages, void* stream);

/* Reconstruct: out row (q, k) (row index q * selected_k + k, 512 BF16 values,
 * contiguous) = dequantized record physical[q, k], tail rotated by freqs row
 * raw[q, k] * 4. A row is zero unless k < lengths[q], 0 <= physical < pool rows
 * and (with freqs) 0 <= raw * 4 < freq_rows. freqs == NULL selects the pre-RoPE
 * reader (raw may be NULL). Strides are in int32 elements. */
int rm_unpack_gather_bf16(const uint8_t* pool, int64_t pool_pages, const int32_t* physical,
                          int64_t physical_stride_q, int64_t physical_stride_k,
                          const int32_t* raw, int64_t raw_stride_q, int64_t raw_stride_k,
                          const int32_t* lengths, int64_t length_stride, int64_t n_queries,
                          int64_t selected_k, const float* freqs, int64_t freq_rows,
                          uint16_t* out, void* stream);

/* rm_unpack_gather_bf16 on a pool of keep_count-survivor records (keep_count
 * 64..448, a multiple of 64; other values give RM_ERR_SHAPE). */
int rm_unpack_gather_bf16_k(const uint8_t* pool, int64_t pool_pages, int keep_count,
                            const int32_t* physical, int64_t physical_stride_q,
                            int64_t physical_stride_k, const int32_t* raw,
                            int64_t raw_stride_q, int64_t raw_stride_k,
                            const int32_t* lengths, int64_t length_stride, int64_t n_queries,
                            int64_t selected_k, const float* freqs, int64_t freq_rows,
                            uint16_t* out, void* stream);

/* rm_unpack_gather_bf16_k reading plane-form buffers of `rows` records
 * (physical entries are plane rows). Planes 8-byte aligned. */
int rm_unpack_gather_bf16_planes(const uint8_t* values, const uint64_t* bitmaps,
                                 const uint8_t* scales, int64_t rows, int keep_count,
                                 const int32_t* physical, int64_t physical_stride_q,
                                 int64_t physical_stride_k, const int32_t* raw,
                                 int64_t raw_stride_q, int64_t raw_stride_k,
                                 const int32_t* lengths, int64_t length_stride, int64_t n_queries,
                                 int64_t selected_k, const float* freqs, int64_t freq_rows,
                                 uint16_t* out, void* stream);

/* Adapter: the rows rm_unpack_gather_bf16 would produce (same gather,
 * validity and RoPE rules; invalid rows are zero rows), each re-encoded as a
 * Native 584-byte record (seven UE8M0/E4M3 NoPE groups from the row's own
 * BF16 values, the tail as BF16, scale row = 7 bytes + a zero pad) at
 * workspace row q * selected_k + k of `native`, a Native page layout of
 * native_pages pages (>= ceil(n_queries * selected_k / 64)). Re-encoding a
 * dequantized Packed row is exact. 256-survivor pools only. */
int rm_packed_to_native(const uint8_t* pool, int64_t pool_pages, const int32_t* physical,
                        int64_t physical_stride_q, int64_t physical_stride_k,
                        const int32_t* raw, int64_t raw_stride_q, int64_t raw_stride_k,
                        const int32_t* lengths, int64_t length_stride, int64_t n_queries,
                        int64_t selected_k, const float* freqs, int64_t freq_rows,
                        uint8_t* native, int64_t native_pages, void* stream);

/* rm_packed_to_native reading plane-form buffers (values [rows, 256]). */
int rm_packed_to_native_planes(const uint8_t* values, const uint64_t* bitmaps,
                               const uint8_t* scales, int64_t rows, const int32_t* physical,
                               int64_t physical_stride_q, int64_t physical_stride_k,
                               const int32_t* raw, int64_t raw_stride_q, int64_t raw_stride_k,
                               const int32_t* lengths, int64_t length_stride, int64_t n_queries,
                               int64_t selected_k, const float* freqs, int64_t freq_rows,
                               uint8_t* native, int64_t native_pages, void* stream);

/* Record transfer between two pools of one format (host-cache backup and
 * restore): for i < n and every layer l < layers, record src_slots[i] of layer
 * l of `src` is copied to record dst_slots[i] of layer l of `dst` -- the whole
 * Packed record (codes, bitmap and scales together; format RM_FORMAT_PACKED
 * with its keep_count) or the Native data row and scale row
 * (RM_FORMAT_NATIVE). Pairs with a slot < 0 or beyond its pool are skipped.
 * Layer l of a pool starts l * layer_bytes after its base. Either pool may be
 * device memory or pinned host memory (hipHostMalloc). 8-byte alignment. */
int rm_copy_records(const uint8_t* src, int64_t src_pages, int64_t src_layer_bytes,
                    const int32_t* src_slots, uint8_t* dst, int64_t dst_pages,
                    int64_t dst_layer_bytes, const int32_t* dst_slots, int64_t n,
                    int64_t layers, int format, int keep_count, void* stream);

/* Split planning for the sparse decode of `tokens` query tokens with `topk`
 * selected records each and `heads` query heads. Writes the number of split-KV
 * partitions and the workspace bytes the decode needs (0 when no split). */
int rm_sparse_decode_workspace(int64_t tokens, int64_t heads, int64_t topk,
                               int32_t* num_splits, size_t* workspace_bytes);

/* Direct packed sparse-MLA decode.
 * q: [batch * q_len, heads, 512] BF16, contiguous; heads a multiple of 16.
 * pool: packed pages. block_table: [batch, block_table_stride] int32; logical
 * record r of request b is pool slot block_table[b, r / 64] * 64 + r % 64.
 * max_blocks: valid columns of the block table. seqlens: [batch] int32 records
 * per request (NULL = unbounded). indices: [batch * q_len, topk] int32 logical
 * records (-1 = padding), topk <= 32768. topk_length: [batch * q_len] int32
 * (NULL = topk).
 * sink: [heads] f32 logits (NULL = no sink). freqs/freq_rows: RoPE table for
 * the stored pre-RoPE tail, row = record * 4, complex64 rows of 32 (cos, sin)
 * pairs; a record whose row r * 4 >= freq_rows contributes nothing.
 * inv_freq: [32] f32 inverse frequencies theta_j, 16-byte aligned (NULL = none).
 * With inv_freq the tail of record r is rotated by the angles RN(RN(4 r) *
 * theta_j), their cos and sin evaluated in the kernel (within a few FP32 ulps
 * of the row 4 r of a table built as polar(1, pos * theta)), and no table row
 * is read; freqs may then be NULL, and when given still bounds the valid
 * records. Neither table nor inv_freq: the tail is used as stored.
 * Output: out [batch * q_len, heads, 512] BF16; lse [batch * q_len, heads] f32,
 * natural log of sum_j exp(l_j) + exp(sink). Invalid entries (k >= length,
 * r < 0, r >= seqlen, unmapped block, row beyond the table) contribute nothing.
 * workspace: rm_sparse_decode_workspace bytes (may be NULL when it reports 0). */
int rm_remnant_sparse_decode_fwd(const uint16_t* q, int64_t batch, int64_t q_len,
                                 int64_t heads, const uint8_t* pool, int64_t pool_pages,
                                 const int32_t* block_table, int64_t block_table_stride,
                                 int64_t max_blocks, const int32_t* seqlens,
                                 const int32_t* indices, int64_t topk,
                                 const int32_t* topk_length, const float* sink,
                                 const float* freqs, int64_t freq_rows, const float* inv_freq,
                                 float softmax_scale, uint16_t* out, float* lse,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* rm_remnant_sparse_decode_swa_fwd on plane-form buffers of pool_rows
 * 256-survivor records (values [rows, 256], bitmaps [rows, 8], scales [rows, 8];
 * pool_rows even, each plane 16-byte aligned): logical record r of request b
 * is plane row block_table[b, r / 64] * 64 + r % 64. swa_topk == 0 attends
 * the C4 list only (the window arguments may then be NULL). */
int rm_remnant_sparse_decode_planes_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* values,
    const uint64_t* bitmaps, const uint8_t* scales, int64_t pool_rows,
    const int32_t* block_table, int64_t block_table_stride, int64_t max_blocks,
    const int32_t* seqlens, const int32_t* indices, int64_t topk, const int32_t* topk_length,
    const uint8_t* swa_pool, int64_t swa_pool_pages, const int32_t* swa_indices,
    int64_t swa_topk, const int32_t* swa_length, const float* sink, const float* freqs,
    int64_t freq_rows, const float* inv_freq, float softmax_scale, uint16_t* out, float* lse,
    void* workspace, size_t workspace_bytes, void* stream);

/* rm_remnant_sparse_decode_swa_fwd without a workspace argument: the split
 * partials live in a 32 MiB device array inside the library (one per GPU,
 * held until the process ends), so the call allocates nothing. No counterpart
 * in the reference: for callers that cannot allocate (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). A call whose split
 * plan needs more than 32 MiB (rm_sparse_decode_workspace_swa) returns
 * RM_ERR_WORKSPACE without launching. The array of the stream's GPU is used;
 * its address is looked up on the first call there, so under HIP graph
 * capture make one eager call on that GPU first. Calls that overlap on one
 * GPU share the array and race; calls on one stream do not. */
int rm_remnant_sparse_decode_swa_noalloc_fwd(
    const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads, const uint8_t* pool,
    int64_t pool_pages, const int32_t* block_table, int64_t block_table_stride,
    int64_t max_blocks, const int32_t* seqlens, const int32_t* indices, int64_t topk,
    const int32_t* topk_length, const uint8_t* swa_pool, int64_t swa_pool_pages,
    const int32_t* swa_indices, int64_t swa_topk, const int32_t* swa_length, const float* sink,
    const float* freqs, int64_t freq_rows, const float* inv_freq, float softmax_scale,
    uint16_t* out, float* lse, void* stream);

/* Native control decode: same contract on 584-byte records (tail already rotated). */
int rm_native_sparse_decode_fwd(const uint16_t* q, int64_t batch, int64_t q_len,
                                int64_t heads, const uint8_t* pool, int64_t pool_pages,
                                const int32_t* block_table, int64_t block_table_stride,
                                int64_t max_blocks, const int32_t* seqlens,
                                const int32_t* indices, int64_t topk,
                                const int32_t* topk_length, const float* sink,
                                float softmax_scale, uint16_t* out, float* lse,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Split planning for the decodes below: as rm_sparse_decode_workspace, plus one
 * partial slot per row for the window rows when swa_topk > 0 (swa_topk <= 512).
 * num_splits counts every slot. */
int rm_sparse_decode_workspace_swa(int64_t tokens, int64_t heads, int64_t topk,
                                   int64_t swa_topk, int32_t* num_splits,
                                   size_t* workspace_bytes);

/* Direct decode with the sliding window: token t attends, in one softmax with
 * the sink, its C4 top-k (as rm_remnant_sparse_decode_fwd) and the window rows
 * swa_indices[t, 0 .. swa_length[t]) (NULL lengths = swa_topk): slots of
 * swa_pool, a Native pool (584-byte records in 64-record pages, tail stored
 * rotated). A slot < 0 or >= swa_pool_pages * 64 contributes nothing.
 * swa_topk <= 512; with window rows topk <= 32256 (63 splits of 512 records,
 * the window taking the 64th partial slot); swa_topk == 0 is
 * rm_remnant_sparse_decode_fwd. */
int rm_remnant_sparse_decode_swa_fwd(const uint16_t* q, int64_t batch, int64_t q_len,
                                     int64_t heads, const uint8_t* pool, int64_t pool_pages,
                                     const int32_t* block_table, int64_t block_table_stride,
                                     int64_t max_blocks, const int32_t* seqlens,
                                     const int32_t* indices, int64_t topk,
                                     const int32_t* topk_length, const uint8_t* swa_pool,
                                     int64_t swa_pool_pages, const int32_t* swa_indices,
                                     int64_t swa_topk, const int32_t* swa_length,
                                     const float* sink, const float* freqs, int64_t freq_rows,
                                     const float* inv_freq, float softmax_scale, uint16_t* out,
                                     float* lse, void* workspace, size_t workspace_bytes,
                                     void* stream);

/* Native control decode with the sliding window (same contract, 584-byte C4 records). */
int rm_native_sparse_decode_swa_fwd(const uint16_t* q, int64_t batch, int64_t q_len,
                                    int64_t heads, const uint8_t* pool, int64_t pool_pages,
                                    const int32_t* block_table, int64_t block_table_stride,
                                    int64_t max_blocks, const int32_t* seqlens,
                                    const int32_t* indices, int64_t topk,
                                    const int32_t* topk_length, const uint8_t* swa_pool,
                                    int64_t swa_pool_pages, const int32_t* swa_indices,
                                    int64_t swa_topk, const int32_t* swa_length,
                                    const float* sink, float softmax_scale, uint16_t* out,
                                    float* lse, void* workspace, size_t workspace_bytes,
                                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* REMNANT_MI355X_H */
