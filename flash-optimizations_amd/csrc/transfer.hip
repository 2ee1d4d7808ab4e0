// Record transfers between two pools of the same format: the host-cache
// (HiCache) backup and restore of latent records.
//
// Reference: the host pool `srt/mem_cache/memory_pool_host.py` and the hybrid
// pool assembler move a record's value, bitmap and scale planes together
// (coordinated transfers, 256 survivors only; third_party/README.md:261). Here
// a Packed record is one contiguous (K + 72)-byte span, so one unit moves all
// three planes; a Native record is its 576-byte data row plus its 8-byte scale
// row. Either pool may live in device memory or in pinned host memory (both
// are addressable from the GPU), so the same kernel backs up (device -> host)
// and restores (host -> device).
//
// One wave per (record, layer): lane l moves 8-byte piece l (and piece 64 + l
// where a record has more than 64 pieces), so a wave issues the whole record
// at once and consecutive waves stream consecutive records.
#include "remnant_device.h"
#include "remnant_mi355x.h"

using namespace rm;

namespace {

constexpr int kWaves = 4;

struct Geometry {
  int64_t page_bytes;
  int data_bytes;   // contiguous bytes at the record's row offset
  int scale_at;     // Native: scale rows' offset in the page (0 for Packed)
  int pieces;       // 8-byte pieces per record, data then (Native) the scale row
};

__device__ __forceinline__ const uint8_t* piece_addr(const uint8_t* pool, int64_t slot, int piece,
                                                     const Geometry& g) {
  const uint8_t* page = pool + (slot >> 6) * g.page_bytes;
  const int row = (int)(slot & 63);
  if (8 * piece < g.data_bytes) return page + (int64_t)row * g.data_bytes + 8 * piece;
  return page + g.scale_at + row * kScaleBytes;  // Native scale row (one piece)
}

__global__ __launch_bounds__(256) void copy_records_kernel(
    const uint8_t* __restrict__ src, int64_t src_rows, int64_t src_layer_bytes,
    const int32_t* __restrict__ src_slots, uint8_t* __restrict__ dst, int64_t dst_rows,
    int64_t dst_layer_bytes, const int32_t* __restrict__ dst_slots, int64_t n, int64_t layers,
    Geometry g) {
  const int lane = wave_lane();
  const int wave = uniform((int)(threadIdx.x >> 6));
  const int64_t units = n * layers;
  for (int64_t u = (int64_t)blockIdx.x * kWaves + wave; u < units;
       u += (int64_t)gridDim.x * kWaves) {
    const int64_t layer = u / n, i = u - layer * n;
    const int64_t s = src_slots[i], d = dst_slots[i];
    if (s < 0 || s >= src_rows || d < 0 || d >= dst_rows) continue;
    const uint8_t* sp = src + layer * src_layer_bytes;
    uint8_t* dp = dst + layer * dst_layer_bytes;
    u32x2 v0 = u32x2{0u, 0u}, v1 = u32x2{0u, 0u};
    const bool has0 = lane < g.pieces, has1 = lane + 64 < g.pieces;
    if (has0) v0 = *(const u32x2*)piece_addr(sp, s, lane, g);
    if (has1) v1 = *(const u32x2*)piece_addr(sp, s, lane + 64, g);
    if (has0) *(u32x2*)piece_addr(dp, d, lane, g) = v0;
    if (has1) *(u32x2*)piece_addr(dp, d, lane + 64, g) = v1;
  }
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace

extern "C" int rm_copy_records(const uint8_t* src, int64_t src_pages, int64_t src_layer_bytes,
                               const int32_t* src_slots, uint8_t* dst, int64_t dst_pages,
                               int64_t dst_layer_bytes, const int32_t* dst_slots, int64_t n,
                               int64_t layers, int format, int keep_count, void* stream) {
  if (n < 0 || layers < 0 || src_pages < 0 || dst_pages < 0) return RM_ERR_SHAPE;
  if (format != RM_FORMAT_PACKED && format != RM_FORMAT_NATIVE) return RM_ERR_DTYPE;
  if (format == RM_FORMAT_PACKED && (keep_count < 64 || keep_count > 448 || keep_count % 64))
    return RM_ERR_SHAPE;
  if (n == 0 || layers == 0) return RM_OK;
  if (!src || !dst || !src_slots || !dst_slots) return RM_ERR_NULL;
  Geometry g;
  if (format == RM_FORMAT_PACKED) {
    g.data_bytes = keep_count + kBitmapBytes + kScaleBytes;
    g.page_bytes = (int64_t)kPageRecords * g.data_bytes;
    g.scale_at = 0;
    g.pieces = g.data_bytes / 8;
  } else {
    g.data_bytes = kNativeDataBytes;
    g.page_bytes = kNativePageBytes;
    g.scale_at = kPageRecords * kNativeDataBytes;
    g.pieces = kNativeDataBytes / 8 + 1;
  }
  // every layer holds the whole page range it is addressed with
  if (layers > 1 && (src_layer_bytes < src_pages * g.page_bytes ||
                     dst_layer_bytes < dst_pages * g.page_bytes))
    return RM_ERR_SHAPE;
  if (!aligned(src, 8) || !aligned(dst, 8) || (src_layer_bytes & 7) || (dst_layer_bytes & 7))
    return RM_ERR_ALIGN;
  int64_t blocks = (n * layers + kWaves - 1) / kWaves;
  if (blocks > 256 * 32) blocks = 256 * 32;
  hipLaunchKernelGGL(copy_records_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, src, src_pages * kPageRecords, src_layer_bytes,
                     src_slots, dst, dst_pages * kPageRecords, dst_layer_bytes, dst_slots, n,
                     layers, g);
  return hipGetLastError() == hipSuccess ? RM_OK : RM_ERR_LAUNCH;
}
