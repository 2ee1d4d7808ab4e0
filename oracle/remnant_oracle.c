/*
 * CPU oracle for the Remnant packed-KV path (test infrastructure only).
 *
 * This file is the checker, never the product: only tests/, the smoke entry
 * and the benchmark's CPU-baseline leg load it. It restates, in plain C with
 * IEEE single precision and no FMA contraction (built with -ffp-contract=off),
 * the DeepSeek-V4 C4 latent codec and the sparse sink attention that the HIP
 * kernels implement.
 *
 * Reference formulas restated here (paths relative to the reference repo):
 *   selection      training/evaluate.py:65-91 (prune topk(|x|, 256, largest=False));
 *                  tie rows asserted in training/tests/test_integration.py:1527-1548
 *   masked RMSNorm training/losses.py:84-89 (m * rsqrt(mean(m^2) + eps) * w -> bf16)
 *   UE8M0 + E4M3   training/losses.py:90-94; closed form at
 *                  training/tests/test_integration.py:1588-1619
 *   record         docs/agents/numerical-and-validation.md:10-12 (256 + 64 + 8 bytes),
 *                  planes at candidate-sglang.patch:900-904; other survivor counts
 *                  64..448 in steps of 64 take count + 72 bytes (same doc, :11-14)
 *   unpack + RoPE  candidate-sglang.patch:502-588 (gather/dequant/zero rows),
 *                  :640-668 (bf16 round, pair rotation, raw*4 frequency row)
 *   native record  training/tests/test_integration.py:361-367 (584-byte layout)
 *   attention      training/losses.py:393-398; sink softmax at
 *                  training/tests/test_integration.py:1620-1635
 *
 * Choices the reference leaves open (its fork sources are not available) are
 * fixed here and mirrored bit-for-bit by the GPU kernels:
 *   - ties at the 256/257 magnitude boundary keep the lower coordinates;
 *   - sum of squares: lane l (coords 8l..8l+7) folds its 8 squares left to
 *     right, then the 64 lane partials are added as a pairwise tree
 *     (distance 1, 2, 4, ... 32);
 *   - rsqrt(v) = RN(1 / RN(sqrt(v))); (m * r) * w are two rounded products;
 *   - bitmap words are MSB-first: coordinate c is bit 63 - (c % 64) of word c/64;
 *   - ties at the K/K+1 boundary of a K-survivor profile likewise;
 *   - a Packed page holds 64 contiguous 328-byte records (codes, bitmap,
 *     scales), or (K + 72)-byte records for K survivors; a Native page holds
 *     the 64 data rows (576 bytes) followed by the 64 scale rows (8 bytes),
 *     matching the reference's Native tail read
 *     native[page, value_base + 448 : value_base + 576] (candidate-sglang.patch:701);
 *   - the RoPE pair rotation is re = RN(RN(xr*c) - RN(xi*s)),
 *     im = RN(RN(xr*s) + RN(xi*c)), on BF16-rounded inputs.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HEAD_DIM 512
#define NOPE_DIM 448
#define ROPE_PAIRS 32
#define KEEP 256
#define GROUP 64
#define NGROUPS 8
#define CODE_BYTES 256
#define BITMAP_BYTES 64
#define DATA_BYTES 320  /* codes + bitmap */
#define SCALE_BYTES 8
#define RECORD_BYTES (DATA_BYTES + SCALE_BYTES) /* 328 */
#define PAGE_RECORDS 64
#define PAGE_BYTES (PAGE_RECORDS * RECORD_BYTES) /* 20992 */
#define NATIVE_DATA_BYTES 576 /* 448 e4m3 + 64 bf16 */
#define NATIVE_PAGE_BYTES (PAGE_RECORDS * (NATIVE_DATA_BYTES + SCALE_BYTES))

/* Threads of the batch loops below (records, rows and tokens are
 * independent; every result is computed the same way on any thread count). */
static int g_threads = 1;
void orc_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int orc_get_threads(void) { return g_threads; }
/* Decode arithmetic: double precision (the default, the checker's) or single
 * precision (a CPU baseline at the GPU kernels' accumulation width). */
static int g_decode_f32 = 0;
void orc_set_decode_f32(int on) { g_decode_f32 = on != 0; }

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* float -> bf16, round to nearest even (NaN kept quiet). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* OCP FP8 E4M3 (e4m3fn) encode with round-to-nearest-even; |q| <= 448. */
uint8_t orc_e4m3_encode(float q) {
    uint32_t b = f2u(q);
    uint8_t sign = (uint8_t)((b >> 24) & 0x80u);
    uint32_t ab = b & 0x7fffffffu;
    float a = u2f(ab);
    if (a < 0x1p-6f) {
        /* subnormal range: value = m * 2^-9, m in 0..8 (8 = smallest normal) */
        int m = (int)nearbyintf(a * 512.0f);
        return (uint8_t)(sign | m);
    }
    uint32_t r = ab + 0x7ffffu + ((ab >> 20) & 1u); /* RNE to 3 mantissa bits */
    int e = (int)(r >> 23) - 127 + 7;
    uint32_t m3 = (r >> 20) & 7u;
    return (uint8_t)(sign | (e << 3) | m3);
}

float orc_e4m3_decode(uint8_t c) {
    int e = (c >> 3) & 15, m = c & 7;
    float v = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return (c & 0x80) ? -v : v;
}

/* UE8M0 exponent: ceil(log2(max(amax, 1e-4) / 448)), evaluated exactly:
 * the smallest e with amax <= 448 * 2^e. */
int orc_ue8m0_exponent(float amax) {
    if (!(amax >= 1e-4f)) return -22;
    uint32_t b = f2u(amax);
    int e = (int)((b >> 23) & 0xffu) - 127;
    return e - 8 + ((b & 0x7fffffu) > 0x600000u ? 1 : 0);
}

static int cmp_desc_u32(const void* a, const void* b) {
    uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return x < y ? 1 : (x > y ? -1 : 0);
}

/* Keep the K largest |x| of 512 (K = 64..448 in steps of 64; 256 is the
 * default profile); ties at the boundary keep lower coordinates. */
void orc_select_keep_k(const float* x, uint8_t* keep, int K) {
    uint32_t key[HEAD_DIM], sorted[HEAD_DIM];
    for (int c = 0; c < HEAD_DIM; ++c) sorted[c] = key[c] = f2u(x[c]) & 0x7fffffffu;
    qsort(sorted, HEAD_DIM, sizeof(uint32_t), cmp_desc_u32);
    uint32_t t = sorted[K - 1];
    int gt = 0;
    for (int c = 0; c < HEAD_DIM; ++c) gt += key[c] > t;
    int ties = K - gt;
    for (int c = 0; c < HEAD_DIM; ++c) {
        if (key[c] > t) keep[c] = 1;
        else if (key[c] == t && ties > 0) { keep[c] = 1; --ties; }
        else keep[c] = 0;
    }
}

void orc_select_keep(const float* x, uint8_t* keep) { orc_select_keep_k(x, keep, KEEP); }

/* Sum of squares in the kernel's fixed order (see header). */
float orc_sumsq(const float* m) {
    float part[64];
    for (int l = 0; l < 64; ++l) {
        float p = m[8 * l] * m[8 * l];
        for (int i = 1; i < 8; ++i) {
            float sq = m[8 * l + i] * m[8 * l + i];
            p = p + sq;
        }
        part[l] = p;
    }
    for (int d = 1; d < 64; d *= 2)
        for (int l = 0; l < 64; l += 2 * d) part[l] = part[l] + part[l + d];
    return part[0];
}

/* r = RN(1 / RN(sqrt(sumsq / 512 + eps))) */
float orc_rms_scale(float sumsq, float eps) {
    float mean = sumsq * (1.0f / 512.0f);
    float v = mean + eps;
    float s = sqrtf(v);
    return 1.0f / s;
}

/* Array forms of the scalar steps, for the checks of the GPU's hardware
 * rounding against this oracle over whole input domains. */
void orc_e4m3_encode_n(const float* q, int64_t n, uint8_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_e4m3_encode(q[i]);
}

/* BF16 of code * 2^(scale_byte - 127), as the unpack computes it. */
void orc_e4m3_dequant_n(const uint8_t* codes, const uint8_t* scale_bytes, int64_t n,
                        uint16_t* out) {
    for (int64_t i = 0; i < n; ++i)
        out[i] = orc_f32_to_bf16(orc_e4m3_decode(codes[i]) *
                                 ldexpf(1.0f, (int)scale_bytes[i] - 127));
}

void orc_rms_scale_n(const float* sumsq, const float* eps, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_rms_scale(sumsq[i], eps[i]);
}

/* Masked RMSNorm -> BF16 (keep may be NULL for the unmasked Native norm). */
void orc_normalize(const float* x, const uint8_t* keep, const float* w, float eps,
                   uint16_t* n) {
    float m[HEAD_DIM];
    for (int c = 0; c < HEAD_DIM; ++c) m[c] = (keep == NULL || keep[c]) ? x[c] : 0.0f;
    float r = orc_rms_scale(orc_sumsq(m), eps);
    for (int c = 0; c < HEAD_DIM; ++c) {
        float y = m[c] * r;
        y = y * w[c];
        n[c] = orc_f32_to_bf16(y);
    }
}

/* Per-64 UE8M0 scale byte and E4M3 codes for groups [g0, g1) of a BF16 row. */
static void quantize_groups(const uint16_t* n, int g0, int g1, uint8_t* codes,
                            uint8_t* scale_bytes) {
    for (int g = g0; g < g1; ++g) {
        float amax = 0.0f;
        for (int c = g * GROUP; c < (g + 1) * GROUP; ++c) {
            float a = fabsf(orc_bf16_to_f32(n[c]));
            if (a > amax) amax = a;
        }
        int e = orc_ue8m0_exponent(amax);
        scale_bytes[g] = (uint8_t)(e + 127);
        float inv = ldexpf(1.0f, -e);
        for (int c = g * GROUP; c < (g + 1) * GROUP; ++c)
            codes[c] = orc_e4m3_encode(orc_bf16_to_f32(n[c]) * inv);
    }
}

/* Dense codec simulation for any mask (training/losses.py:74-95 semantics):
 * masked RMSNorm -> BF16 -> per-64 UE8M0/E4M3 -> decoded BF16 (pre-RoPE),
 * pruned coordinates zero. Used for the closed-form checks at any budget. */
void orc_simulate_rows(const float* x, const uint8_t* keep, const float* w, float eps,
                       int64_t rows, uint16_t* out) {
    for (int64_t r = 0; r < rows; ++r) {
        uint16_t n[HEAD_DIM];
        uint8_t codes[HEAD_DIM], sb[NGROUPS];
        orc_normalize(x + r * HEAD_DIM, keep + r * HEAD_DIM, w + r * HEAD_DIM, eps, n);
        quantize_groups(n, 0, NGROUPS, codes, sb);
        for (int c = 0; c < HEAD_DIM; ++c) {
            float v = orc_e4m3_decode(codes[c]) * ldexpf(1.0f, (int)sb[c / GROUP] - 127);
            out[r * HEAD_DIM + c] = keep[r * HEAD_DIM + c] ? orc_f32_to_bf16(v) : 0;
        }
    }
}

/* Pack one record with K survivors: data = K codes (ascending coordinate) +
 * 8 MSB-first uint64 bitmap words (little-endian bytes); scales = 8 UE8M0
 * bytes. A K-survivor record is K + 72 bytes (codes, bitmap, scales). */
void orc_pack_row_k(const float* x, const float* w, float eps, int K, uint8_t* data,
                    uint8_t* scales, uint16_t* normalized_out, uint8_t* keep_out) {
    uint8_t keep[HEAD_DIM], codes[HEAD_DIM];
    uint16_t n[HEAD_DIM];
    orc_select_keep_k(x, keep, K);
    orc_normalize(x, keep, w, eps, n);
    quantize_groups(n, 0, NGROUPS, codes, scales);
    int rank = 0;
    memset(data, 0, K + BITMAP_BYTES);
    for (int c = 0; c < HEAD_DIM; ++c) {
        if (!keep[c]) continue;
        data[rank++] = codes[c];
        int word = c / 64, bit = 63 - (c % 64);
        data[K + word * 8 + bit / 8] |= (uint8_t)(1u << (bit % 8));
    }
    if (normalized_out) memcpy(normalized_out, n, sizeof(n));
    if (keep_out) memcpy(keep_out, keep, sizeof(keep));
}

void orc_pack_row(const float* x, const float* w, float eps, uint8_t* data,
                  uint8_t* scales, uint16_t* normalized_out, uint8_t* keep_out) {
    orc_pack_row_k(x, w, eps, KEEP, data, scales, normalized_out, keep_out);
}

static inline int64_t page_of(int64_t slot) { return slot / PAGE_RECORDS; }

/* Record bytes and page bytes of the K-survivor Packed format. */
static inline int64_t record_bytes_k(int K) { return K + BITMAP_BYTES + SCALE_BYTES; }
static inline int64_t page_bytes_k(int K) { return PAGE_RECORDS * record_bytes_k(K); }

/* Pack rows into the paged pool at dst_slot[i] (negative slots are skipped).
 * With more than one thread the slots must be distinct. */
void orc_pack_rows_paged_k(const float* x, const float* w, float eps, int K,
                           const int32_t* slot, int64_t rows, uint8_t* pool,
                           int64_t pool_pages) {
    const int64_t rb = record_bytes_k(K), pb = page_bytes_k(K);
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t i = 0; i < rows; ++i) {
        int64_t s = slot[i];
        if (s < 0 || s >= pool_pages * PAGE_RECORDS) continue;
        uint8_t* rec = pool + page_of(s) * pb + (s % PAGE_RECORDS) * rb;
        orc_pack_row_k(x + i * HEAD_DIM, w, eps, K, rec, rec + K + BITMAP_BYTES, NULL, NULL);
    }
}

void orc_pack_rows_paged(const float* x, const float* w, float eps, const int32_t* slot,
                         int64_t rows, uint8_t* pool, int64_t pool_pages) {
    orc_pack_rows_paged_k(x, w, eps, KEEP, slot, rows, pool, pool_pages);
}

/* Dequantize one K-survivor record to pre-RoPE BF16 (exact). */
void orc_unpack_row_k(const uint8_t* data, const uint8_t* scales, int K, uint16_t* out) {
    int rank = 0;
    for (int c = 0; c < HEAD_DIM; ++c) {
        int word = c / 64, bit = 63 - (c % 64);
        int kept = (data[K + word * 8 + bit / 8] >> (bit % 8)) & 1;
        if (!kept) { out[c] = 0; continue; }
        float v = orc_e4m3_decode(data[rank++]) * ldexpf(1.0f, (int)scales[c / GROUP] - 127);
        out[c] = orc_f32_to_bf16(v);
    }
}

void orc_unpack_row(const uint8_t* data, const uint8_t* scales, uint16_t* out) {
    orc_unpack_row_k(data, scales, KEEP, out);
}

/* In-place tail rotation of a BF16 row with one complex frequency row
 * (32 interleaved (cos, sin) float pairs). */
void orc_rope_tail(uint16_t* row, const float* freq) {
    for (int j = 0; j < ROPE_PAIRS; ++j) {
        float xr = orc_bf16_to_f32(row[NOPE_DIM + 2 * j]);
        float xi = orc_bf16_to_f32(row[NOPE_DIM + 2 * j + 1]);
        float c = freq[2 * j], s = freq[2 * j + 1];
        float a = xr * c, b = xi * s, re = a - b;
        float d = xr * s, e = xi * c, im = d + e;
        row[NOPE_DIM + 2 * j] = orc_f32_to_bf16(re);
        row[NOPE_DIM + 2 * j + 1] = orc_f32_to_bf16(im);
    }
}

/* unpack_gather_bf16 (candidate-sglang.patch:427-480, 502-668): row (q, k)
 * gathers pool slot physical[q, k]; it is zero unless k < lengths[q],
 * 0 <= physical < pool rows and, with a frequency table, 0 <= raw*4 < freq_rows.
 * freqs == NULL selects the pre-RoPE reader (raw unused). K is the pool's
 * survivor count (its records are K + 72 bytes). */
void orc_unpack_gather_k(const uint8_t* pool, int64_t pool_pages, int K,
                         const int32_t* physical, int64_t ps_q, int64_t ps_k,
                         const int32_t* raw, int64_t rs_q, int64_t rs_k,
                         const int32_t* lengths, int64_t ls, int64_t nq, int64_t nk,
                         const float* freqs, int64_t freq_rows, uint16_t* out) {
    int64_t rows = pool_pages * PAGE_RECORDS;
    const int64_t rb = record_bytes_k(K), pb = page_bytes_k(K);
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t qk = 0; qk < nq * nk; ++qk) {
        const int64_t q = qk / nk, k = qk % nk;
        uint16_t* o = out + (q * nk + k) * HEAD_DIM;
        int64_t p = physical[q * ps_q + k * ps_k];
        int64_t r = raw ? raw[q * rs_q + k * rs_k] : 0;
        int valid = k < lengths[q * ls] && p >= 0 && p < rows;
        if (freqs) valid = valid && r >= 0 && r * 4 < freq_rows;
        if (!valid) { memset(o, 0, HEAD_DIM * 2); continue; }
        const uint8_t* rec = pool + page_of(p) * pb + (p % PAGE_RECORDS) * rb;
        orc_unpack_row_k(rec, rec + K + BITMAP_BYTES, K, o);
        if (freqs) orc_rope_tail(o, freqs + r * 4 * ROPE_PAIRS * 2);
    }
}

void orc_unpack_gather(const uint8_t* pool, int64_t pool_pages, const int32_t* physical,
                       int64_t ps_q, int64_t ps_k, const int32_t* raw, int64_t rs_q,
                       int64_t rs_k, const int32_t* lengths, int64_t ls, int64_t nq,
                       int64_t nk, const float* freqs, int64_t freq_rows, uint16_t* out) {
    orc_unpack_gather_k(pool, pool_pages, KEEP, physical, ps_q, ps_k, raw, rs_q, rs_k, lengths,
                        ls, nq, nk, freqs, freq_rows, out);
}

/* Native 584-byte record: unpruned RMSNorm -> BF16; nope groups 0..6 as
 * UE8M0/E4M3 (448 code bytes); tail rotated BF16 (128 bytes); scale row =
 * 7 UE8M0 bytes + one zero pad byte. freq may be NULL (no rotation). */
void orc_native_pack_row(const float* x, const float* w, float eps, const float* freq,
                         uint8_t* data, uint8_t* scales) {
    uint16_t n[HEAD_DIM];
    uint8_t codes[HEAD_DIM], sb[NGROUPS];
    orc_normalize(x, NULL, w, eps, n);
    quantize_groups(n, 0, NOPE_DIM / GROUP, codes, sb);
    if (freq) orc_rope_tail(n, freq);
    memcpy(data, codes, NOPE_DIM);
    memcpy(data + NOPE_DIM, n + NOPE_DIM, (HEAD_DIM - NOPE_DIM) * 2);
    memcpy(scales, sb, NOPE_DIM / GROUP);
    scales[NOPE_DIM / GROUP] = 0;
}

/* Native record of a dense BF16 row (the dense BF16 -> Native conversion
 * `_bf16_to_native_kernel` of the reference's Triton decode, launch list in
 * benchmarks/microbench/dsv4-flash-decode-store/profiling/h64_b16_k512/
 * metrics.json; the CUDA Adapter, third_party/README.md:259): nope groups 0..6 as
 * UE8M0/E4M3 from the row's own BF16 values, the tail copied as stored, scale
 * row = 7 bytes + one zero pad byte. A zero row gives zero codes and scale
 * bytes 105 (the 1e-4 amax floor). */
void orc_native_encode_row(const uint16_t* row, uint8_t* data, uint8_t* scales) {
    uint8_t codes[HEAD_DIM], sb[NGROUPS];
    quantize_groups(row, 0, NOPE_DIM / GROUP, codes, sb);
    memcpy(data, codes, NOPE_DIM);
    memcpy(data + NOPE_DIM, row + NOPE_DIM, (HEAD_DIM - NOPE_DIM) * 2);
    memcpy(scales, sb, NOPE_DIM / GROUP);
    scales[NOPE_DIM / GROUP] = 0;
}

void orc_native_pack_rows_paged(const float* x, const float* w, float eps,
                                const int32_t* slot, const int32_t* position,
                                const float* freqs, int64_t freq_rows, int64_t rows,
                                uint8_t* pool, int64_t pool_pages) {
    for (int64_t i = 0; i < rows; ++i) {
        int64_t s = slot[i];
        if (s < 0 || s >= pool_pages * PAGE_RECORDS) continue;
        const float* f = NULL;
        if (freqs) {
            int64_t r = position[i];
            if (r < 0 || r * 4 >= freq_rows) continue;
            f = freqs + r * 4 * ROPE_PAIRS * 2;
        }
        uint8_t* page = pool + page_of(s) * NATIVE_PAGE_BYTES;
        int in = (int)(s % PAGE_RECORDS);
        orc_native_pack_row(x + i * HEAD_DIM, w, eps, f, page + in * NATIVE_DATA_BYTES,
                            page + PAGE_RECORDS * NATIVE_DATA_BYTES + in * SCALE_BYTES);
    }
}

void orc_native_unpack_row(const uint8_t* data, const uint8_t* scales, uint16_t* out) {
    for (int c = 0; c < NOPE_DIM; ++c)
        out[c] = orc_f32_to_bf16(orc_e4m3_decode(data[c]) *
                                 ldexpf(1.0f, (int)scales[c / GROUP] - 127));
    memcpy(out + NOPE_DIM, data + NOPE_DIM, (HEAD_DIM - NOPE_DIM) * 2);
}

/* Gather the K rows one decode token attends to, through the block table:
 * logical record r of request b lives in page block_table[b, r / 64], slot
 * r % 64. valid[k] = 0 for k >= length, r < 0, r >= seqlen, unmapped pages or
 * (packed with RoPE) r*4 >= freq_rows. packed != 0 selects the 328-byte
 * format (tail RoPE from freqs); otherwise the Native 584-byte format. */
void orc_decode_gather(const uint8_t* pool, int64_t pool_pages, int packed,
                       const int32_t* block_table, int64_t bt_stride, int64_t max_blocks,
                       int64_t seqlen, const int32_t* indices, int64_t nk, int64_t length,
                       const float* freqs, int64_t freq_rows, uint16_t* rows,
                       uint8_t* valid) {
    for (int64_t k = 0; k < nk; ++k) {
        uint16_t* o = rows + k * HEAD_DIM;
        int64_t r = indices[k];
        int ok = k < length && r >= 0 && r < seqlen && r / PAGE_RECORDS < max_blocks;
        int64_t page = ok ? block_table[(r / PAGE_RECORDS) * bt_stride] : -1;
        ok = ok && page >= 0 && page < pool_pages;
        if (ok && packed && freqs) ok = r * 4 < freq_rows;
        valid[k] = (uint8_t)ok;
        if (!ok) { memset(o, 0, HEAD_DIM * 2); continue; }
        int in = (int)(r % PAGE_RECORDS);
        if (packed) {
            const uint8_t* rec = pool + page * PAGE_BYTES + in * RECORD_BYTES;
            orc_unpack_row(rec, rec + DATA_BYTES, o);
            if (freqs) orc_rope_tail(o, freqs + r * 4 * ROPE_PAIRS * 2);
        } else {
            const uint8_t* pg = pool + page * NATIVE_PAGE_BYTES;
            orc_native_unpack_row(pg + in * NATIVE_DATA_BYTES,
                                  pg + PAGE_RECORDS * NATIVE_DATA_BYTES + in * SCALE_BYTES, o);
        }
    }
}

/* Sparse sink attention for one token in double precision:
 * logits l_j = (q_h . K_j) * scale over valid rows; Z = sum exp(l_j) + exp(sink_h);
 * out_h = sum_j exp(l_j) K_j / Z; lse_h = log Z (sink == NULL: no sink term).
 * With no valid row and no sink, out = 0 and lse = -inf. V = K (same row). */
/* The same in single precision (logits, weights, sums and output in float). */
static void sink_attention_head_f32(const uint16_t* qh, const uint16_t* rows,
                                    const uint8_t* valid, int64_t nk, const float* sink_h,
                                    float scale, double* logit_scratch, double* oh,
                                    double* lse_h) {
    float* logit = (float*)logit_scratch;
    float qf[HEAD_DIM], of[HEAD_DIM];
    for (int c = 0; c < HEAD_DIM; ++c) qf[c] = orc_bf16_to_f32(qh[c]);
    float mx = sink_h ? *sink_h : -INFINITY;
    for (int64_t k = 0; k < nk; ++k) {
        if (!valid[k]) continue;
        float acc = 0.0f;
        const uint16_t* kr = rows + k * HEAD_DIM;
        for (int c = 0; c < HEAD_DIM; ++c) acc += qf[c] * orc_bf16_to_f32(kr[c]);
        logit[k] = acc * scale;
        if (logit[k] > mx) mx = logit[k];
    }
    for (int c = 0; c < HEAD_DIM; ++c) oh[c] = 0.0;
    if (mx == -INFINITY) { *lse_h = -INFINITY; return; }
    for (int c = 0; c < HEAD_DIM; ++c) of[c] = 0.0f;
    float z = sink_h ? expf(*sink_h - mx) : 0.0f;
    for (int64_t k = 0; k < nk; ++k) {
        if (!valid[k]) continue;
        const float p = expf(logit[k] - mx);
        z += p;
        const uint16_t* kr = rows + k * HEAD_DIM;
        for (int c = 0; c < HEAD_DIM; ++c) of[c] += p * orc_bf16_to_f32(kr[c]);
    }
    for (int c = 0; c < HEAD_DIM; ++c) oh[c] = (double)(of[c] / z);
    *lse_h = (double)(mx + logf(z));
}

/* One head of orc_sink_attention (logit: nk doubles of scratch). */
static void sink_attention_head(const uint16_t* qh, const uint16_t* rows, const uint8_t* valid,
                                int64_t nk, const float* sink_h, float scale, double* logit,
                                double* oh, double* lse_h) {
    if (g_decode_f32) {
        sink_attention_head_f32(qh, rows, valid, nk, sink_h, scale, logit, oh, lse_h);
        return;
    }
    double mx = sink_h ? (double)*sink_h : -INFINITY;
    for (int64_t k = 0; k < nk; ++k) {
        if (!valid[k]) continue;
        double acc = 0.0;
        const uint16_t* kr = rows + k * HEAD_DIM;
        for (int c = 0; c < HEAD_DIM; ++c)
            acc += (double)orc_bf16_to_f32(qh[c]) * (double)orc_bf16_to_f32(kr[c]);
        logit[k] = acc * (double)scale;
        if (logit[k] > mx) mx = logit[k];
    }
    for (int c = 0; c < HEAD_DIM; ++c) oh[c] = 0.0;
    if (mx == -INFINITY) { *lse_h = -INFINITY; return; }
    double z = sink_h ? exp((double)*sink_h - mx) : 0.0;
    for (int64_t k = 0; k < nk; ++k) {
        if (!valid[k]) continue;
        double p = exp(logit[k] - mx);
        z += p;
        const uint16_t* kr = rows + k * HEAD_DIM;
        for (int c = 0; c < HEAD_DIM; ++c) oh[c] += p * (double)orc_bf16_to_f32(kr[c]);
    }
    for (int c = 0; c < HEAD_DIM; ++c) oh[c] /= z;
    *lse_h = mx + log(z);
}

void orc_sink_attention(const uint16_t* q, int64_t heads, const uint16_t* rows,
                        const uint8_t* valid, int64_t nk, const float* sink, float scale,
                        double* out, double* lse) {
    double* logit = (double*)malloc(sizeof(double) * (nk > 0 ? nk : 1));
    for (int64_t h = 0; h < heads; ++h)
        sink_attention_head(q + h * HEAD_DIM, rows, valid, nk, sink ? sink + h : NULL, scale,
                            logit, out + h * HEAD_DIM, lse + h);
    free(logit);
}

/* Whole decode step: tokens t = b * q_len + s share request b's block table. */
void orc_sparse_decode(const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads,
                       const uint8_t* pool, int64_t pool_pages, int packed,
                       const int32_t* block_table, int64_t bt_stride, int64_t max_blocks,
                       const int32_t* seqlens, const int32_t* indices, int64_t topk,
                       const int32_t* topk_length, const float* sink, const float* freqs,
                       int64_t freq_rows, float scale, double* out, double* lse) {
    const int64_t tokens = batch * q_len;
    if (tokens < g_threads) {
        /* few tokens (batch 1): per token, the gather in record chunks and the
         * heads on all threads -- the same arithmetic per head as below */
        const int64_t nk = topk > 0 ? topk : 1;
        uint16_t* rows = (uint16_t*)malloc(sizeof(uint16_t) * HEAD_DIM * nk);
        uint8_t* valid = (uint8_t*)malloc(nk);
        for (int64_t t = 0; t < tokens; ++t) {
            const int64_t b = t / q_len;
            const int64_t len = topk_length ? topk_length[t] : topk;
            const int64_t chunk = 64, chunks = (topk + chunk - 1) / chunk;
#pragma omp parallel for num_threads(g_threads) schedule(dynamic)
            for (int64_t c = 0; c < chunks; ++c) {
                const int64_t k0 = c * chunk, k1 = k0 + chunk < topk ? k0 + chunk : topk;
                orc_decode_gather(pool, pool_pages, packed, block_table + b * bt_stride, 1,
                                  max_blocks, seqlens ? seqlens[b] : INT64_MAX,
                                  indices + t * topk + k0, k1 - k0, len - k0, freqs, freq_rows,
                                  rows + k0 * HEAD_DIM, valid + k0);
            }
#pragma omp parallel num_threads(g_threads)
            {
                double* logit = (double*)malloc(sizeof(double) * nk);
#pragma omp for schedule(dynamic)
                for (int64_t h = 0; h < heads; ++h)
                    sink_attention_head(q + (t * heads + h) * HEAD_DIM, rows, valid, topk,
                                        sink ? sink + h : NULL, scale, logit,
                                        out + (t * heads + h) * HEAD_DIM, lse + t * heads + h);
                free(logit);
            }
        }
        free(rows);
        free(valid);
        return;
    }
#pragma omp parallel num_threads(g_threads)
    {
        uint16_t* rows = (uint16_t*)malloc(sizeof(uint16_t) * HEAD_DIM * (topk > 0 ? topk : 1));
        uint8_t* valid = (uint8_t*)malloc(topk > 0 ? topk : 1);
#pragma omp for schedule(dynamic)
        for (int64_t t = 0; t < batch * q_len; ++t) {
            const int64_t b = t / q_len;
            int64_t len = topk_length ? topk_length[t] : topk;
            orc_decode_gather(pool, pool_pages, packed, block_table + b * bt_stride, 1,
                              max_blocks, seqlens ? seqlens[b] : INT64_MAX,
                              indices + t * topk, topk, len, freqs, freq_rows, rows, valid);
            orc_sink_attention(q + t * heads * HEAD_DIM, heads, rows, valid, topk, sink,
                               scale, out + t * heads * HEAD_DIM, lse + t * heads);
        }
        free(rows);
        free(valid);
    }
}

/* SWA rows of one token: the rows lie in a Native pool (64-record pages) at
 * physical slots swa_slots[k]; valid[k] = 0 for k >= length or a slot outside
 * the pool. Rows are stored with the tail already rotated. */
void orc_swa_gather(const uint8_t* swa_pool, int64_t swa_pages, const int32_t* swa_slots,
                    int64_t nk, int64_t length, uint16_t* rows, uint8_t* valid) {
    for (int64_t k = 0; k < nk; ++k) {
        uint16_t* o = rows + k * HEAD_DIM;
        int64_t sl = swa_slots[k];
        int ok = k < length && sl >= 0 && sl < swa_pages * PAGE_RECORDS;
        valid[k] = (uint8_t)ok;
        if (!ok) { memset(o, 0, HEAD_DIM * 2); continue; }
        const uint8_t* pg = swa_pool + page_of(sl) * NATIVE_PAGE_BYTES;
        int in = (int)(sl % PAGE_RECORDS);
        orc_native_unpack_row(pg + in * NATIVE_DATA_BYTES,
                              pg + PAGE_RECORDS * NATIVE_DATA_BYTES + in * SCALE_BYTES, o);
    }
}

/* Decode step with the sliding-window rows attended jointly (training/losses.py:
 * 393-398: softmax over cat(swa rows, C4 rows) plus the sink): token t attends
 * its swa_topk SWA slots (swa_length[t] of them valid; NULL = all) and its
 * C4 top-k exactly as orc_sparse_decode does, in one softmax. */
void orc_sparse_decode_swa(const uint16_t* q, int64_t batch, int64_t q_len, int64_t heads,
                           const uint8_t* pool, int64_t pool_pages, int packed,
                           const int32_t* block_table, int64_t bt_stride, int64_t max_blocks,
                           const int32_t* seqlens, const int32_t* indices, int64_t topk,
                           const int32_t* topk_length, const uint8_t* swa_pool,
                           int64_t swa_pages, const int32_t* swa_indices, int64_t swa_topk,
                           const int32_t* swa_length, const float* sink, const float* freqs,
                           int64_t freq_rows, float scale, double* out, double* lse) {
    int64_t nk = swa_topk + topk;
    uint16_t* rows = (uint16_t*)malloc(sizeof(uint16_t) * HEAD_DIM * (nk > 0 ? nk : 1));
    uint8_t* valid = (uint8_t*)malloc(nk > 0 ? nk : 1);
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t s = 0; s < q_len; ++s) {
            int64_t t = b * q_len + s;
            int64_t len = topk_length ? topk_length[t] : topk;
            int64_t swa_len = swa_length ? swa_length[t] : swa_topk;
            orc_swa_gather(swa_pool, swa_pages, swa_indices + t * swa_topk, swa_topk, swa_len,
                           rows, valid);
            orc_decode_gather(pool, pool_pages, packed, block_table + b * bt_stride, 1,
                              max_blocks, seqlens ? seqlens[b] : INT64_MAX,
                              indices + t * topk, topk, len, freqs, freq_rows,
                              rows + swa_topk * HEAD_DIM, valid + swa_topk);
            orc_sink_attention(q + t * heads * HEAD_DIM, heads, rows, valid, nk, sink, scale,
                               out + t * heads * HEAD_DIM, lse + t * heads);
        }
    free(rows);
    free(valid);
}

/* Adapter (Packed -> Native workspace, third_party/README.md:259, 289): row
 * (q, k) of unpack_gather_bf16 (same gather, validity and RoPE rules; invalid
 * rows are zero rows) re-encoded as a Native record at workspace row
 * q * nk + k (page row / 64, slot row % 64 of a Native page layout). */
void orc_packed_to_native(const uint8_t* pool, int64_t pool_pages, const int32_t* physical,
                          int64_t ps_q, int64_t ps_k, const int32_t* raw, int64_t rs_q,
                          int64_t rs_k, const int32_t* lengths, int64_t ls, int64_t nq,
                          int64_t nk, const float* freqs, int64_t freq_rows, uint8_t* out) {
    uint16_t* rows = (uint16_t*)malloc(sizeof(uint16_t) * HEAD_DIM * (nq * nk > 0 ? nq * nk : 1));
    orc_unpack_gather(pool, pool_pages, physical, ps_q, ps_k, raw, rs_q, rs_k, lengths, ls, nq,
                      nk, freqs, freq_rows, rows);
    for (int64_t i = 0; i < nq * nk; ++i) {
        uint8_t* pg = out + page_of(i) * NATIVE_PAGE_BYTES;
        int in = (int)(i % PAGE_RECORDS);
        orc_native_encode_row(rows + i * HEAD_DIM, pg + in * NATIVE_DATA_BYTES,
                              pg + PAGE_RECORDS * NATIVE_DATA_BYTES + in * SCALE_BYTES);
    }
    free(rows);
}
