// Cluster permute / inverse permute of [BH, S, row] tensors (HBM-bound row gathers).
//
// Replaces permute_tensor_by_labels_triton / apply_inverse_permutation_triton /
// permute_concatenated_tensors_by_labels_triton (reference
// src/sparsepr/kernels/triton/permute.py:126-172, :235-274, :175-232).
//
// One 16-byte vector per thread per step, UNROLL independent vectors in flight,
// 2-D grid (x: vectors within one bh, y: bh) so all index math is 32-bit.
// Index values outside [0, S) are never dereferenced: a gather writes zeros, a
// scatter drops the row.
#include "spr_common.h"

namespace {

enum { MODE_GATHER = 0, MODE_SCATTER = 1, MODE_CONCAT = 2 };

template <typename V, int UNROLL, int MODE>
__global__ __launch_bounds__(256) void permute_rows_kernel(const V* __restrict__ src,
                                                           const V* __restrict__ suffix,
                                                           const int32_t* __restrict__ idx,
                                                           V* __restrict__ dst, uint32_t src_rows,
                                                           uint32_t dst_rows, uint32_t prefix_rows,
                                                           uint32_t vec_per_row, uint64_t src_bh) {
  // src_bh: vectors from one head's source rows to the next (MODE_GATHER / MODE_SCATTER)
  // MODE_GATHER / MODE_CONCAT walk the destination rows (idx has dst_rows
  // entries per bh); MODE_SCATTER walks the source rows (idx has src_rows).
  const uint32_t walk_rows = (MODE == MODE_SCATTER) ? src_rows : dst_rows;
  const uint32_t per_bh = walk_rows * vec_per_row;
  const uint64_t bh = blockIdx.y;
  const int32_t* idx_bh = idx + bh * walk_rows;
  const uint32_t base = blockIdx.x * (256u * UNROLL) + threadIdx.x;
  V vals[UNROLL];
  uint64_t dst_off[UNROLL];
  bool live[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const uint32_t g = base + u * 256u;
    live[u] = g < per_bh;
    const uint32_t row = live[u] ? g / vec_per_row : 0u;
    const uint32_t v = g - row * vec_per_row;
    const uint32_t r = static_cast<uint32_t>(live[u] ? idx_bh[row] : 0);
    if (MODE == MODE_GATHER) {
      const bool valid = live[u] && r < src_rows;
      dst_off[u] = bh * per_bh + g;
      vals[u] = valid ? src[bh * src_bh + static_cast<uint64_t>(r) * vec_per_row + v] : V{};
    } else if (MODE == MODE_SCATTER) {
      vals[u] = live[u] ? src[bh * src_bh + g] : V{};
      dst_off[u] = (bh * dst_rows + r) * vec_per_row + v;
      live[u] = live[u] && r < dst_rows;
    } else {
      const bool valid = live[u] && r < src_rows;
      dst_off[u] = bh * per_bh + g;
      if (!valid) {
        vals[u] = V{};
      } else if (r < prefix_rows) {
        vals[u] = src[(bh * prefix_rows + r) * vec_per_row + v];
      } else {
        const uint32_t suffix_rows = src_rows - prefix_rows;
        vals[u] = suffix[(bh * suffix_rows + (r - prefix_rows)) * vec_per_row + v];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    if (live[u]) dst[dst_off[u]] = vals[u];
  }
}

template <int MODE>
int launch_permute(const void* src, const void* suffix, const int32_t* idx, void* dst, int64_t bh,
                   int64_t src_rows, int64_t dst_rows, int64_t prefix_rows, int64_t row_bytes,
                   hipStream_t stream, const char* name, int64_t src_head_bytes = -1) {
  // src_head_bytes: bytes from one head's source rows to the next (-1: packed, src_rows rows)
  SPR_REQUIRE(bh >= 0 && src_rows >= 0 && dst_rows >= 0, "%s: negative size", name);
  const int64_t walk_rows = (MODE == MODE_SCATTER) ? src_rows : dst_rows;
  if (bh == 0 || walk_rows == 0 || row_bytes == 0) return SPR_OK;
  SPR_REQUIRE(src && idx && dst, "%s: null pointer", name);
  SPR_REQUIRE(bh <= 65535, "%s: bh=%lld exceeds 65535", name, (long long)bh);
  SPR_REQUIRE(row_bytes % 2 == 0, "%s: row bytes %lld not a multiple of 2", name, (long long)row_bytes);
  if (src_head_bytes == -1) src_head_bytes = src_rows * row_bytes;
  SPR_REQUIRE(src_head_bytes >= src_rows * row_bytes, "%s: source head stride %lld below %lld rows of %lld bytes",
              name, (long long)src_head_bytes, (long long)src_rows, (long long)row_bytes);
  auto aligned = [&](uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(src) % a == 0) && (reinterpret_cast<uintptr_t>(dst) % a == 0) &&
           (suffix == nullptr || reinterpret_cast<uintptr_t>(suffix) % a == 0) &&
           static_cast<uintptr_t>(src_head_bytes) % a == 0;
  };
  const bool wide = (row_bytes % 16 == 0) && aligned(16);
  const bool word = !wide && (row_bytes % 4 == 0) && aligned(4);
  const int64_t vec = wide ? 16 : (word ? 4 : 2);
  const int64_t vpr = row_bytes / vec;
  const int64_t biggest = src_rows > dst_rows ? src_rows : dst_rows;
  SPR_REQUIRE(biggest * vpr < (int64_t(1) << 31), "%s: %lld rows of %lld bytes exceed the per-head limit",
              name, (long long)biggest, (long long)row_bytes);
  constexpr int UNROLL = 4;
  const int64_t per_bh = walk_rows * vpr;
  dim3 grid(static_cast<uint32_t>(spr::ceil_div(per_bh, 256 * UNROLL)), static_cast<uint32_t>(bh));
  if (wide) {
    permute_rows_kernel<spr::u32x4, UNROLL, MODE><<<grid, 256, 0, stream>>>(
        static_cast<const spr::u32x4*>(src), static_cast<const spr::u32x4*>(suffix), idx,
        static_cast<spr::u32x4*>(dst), static_cast<uint32_t>(src_rows), static_cast<uint32_t>(dst_rows),
        static_cast<uint32_t>(prefix_rows), static_cast<uint32_t>(vpr), static_cast<uint64_t>(src_head_bytes / vec));
  } else if (word) {
    permute_rows_kernel<uint32_t, UNROLL, MODE><<<grid, 256, 0, stream>>>(
        static_cast<const uint32_t*>(src), static_cast<const uint32_t*>(suffix), idx,
        static_cast<uint32_t*>(dst), static_cast<uint32_t>(src_rows), static_cast<uint32_t>(dst_rows),
        static_cast<uint32_t>(prefix_rows), static_cast<uint32_t>(vpr), static_cast<uint64_t>(src_head_bytes / vec));
  } else {
    permute_rows_kernel<uint16_t, UNROLL, MODE><<<grid, 256, 0, stream>>>(
        static_cast<const uint16_t*>(src), static_cast<const uint16_t*>(suffix), idx,
        static_cast<uint16_t*>(dst), static_cast<uint32_t>(src_rows), static_cast<uint32_t>(dst_rows),
        static_cast<uint32_t>(prefix_rows), static_cast<uint32_t>(vpr), static_cast<uint64_t>(src_head_bytes / vec));
  }
  SPR_LAUNCHED(name);
  return SPR_OK;
}

}  // namespace

// dst[b, s, :] = src[b, idx[b, s], :]
extern "C" int spr_permute_rows(const void* src, const int32_t* idx, void* dst, int64_t bh, int64_t rows,
                                int64_t row_bytes, hipStream_t stream) {
  return launch_permute<MODE_GATHER>(src, nullptr, idx, dst, bh, rows, rows, 0, row_bytes, stream,
                                     "spr_permute_rows");
}

// dst[b, idx[b, s], :] = src[b, s, :]
extern "C" int spr_inverse_permute_rows(const void* src, const int32_t* idx, void* dst, int64_t bh,
                                        int64_t rows, int64_t row_bytes, hipStream_t stream) {
  return launch_permute<MODE_SCATTER>(src, nullptr, idx, dst, bh, rows, rows, 0, row_bytes, stream,
                                      "spr_inverse_permute_rows");
}

// spr_inverse_permute_rows with head b's source rows starting src_head_bytes after head
// b - 1's (a slice of the rows of a larger packed tensor, read in place); the stride is
// explicit, at least rows * row_bytes (no value stands for "packed").
extern "C" int spr_inverse_permute_rows_strided(const void* src, int64_t src_head_bytes, const int32_t* idx, void* dst,
                                                int64_t bh, int64_t rows, int64_t row_bytes, hipStream_t stream) {
  SPR_REQUIRE(src_head_bytes >= 0 && src_head_bytes >= rows * row_bytes,
              "spr_inverse_permute_rows_strided: source head stride %lld below %lld rows of %lld bytes",
              (long long)src_head_bytes, (long long)rows, (long long)row_bytes);
  return launch_permute<MODE_SCATTER>(src, nullptr, idx, dst, bh, rows, rows, 0, row_bytes, stream,
                                      "spr_inverse_permute_rows_strided", src_head_bytes);
}

// dst[b, s, :] = cat(prefix[b], suffix[b])[idx[b, s], :]
extern "C" int spr_permute_concat_rows(const void* prefix, const void* suffix, const int32_t* idx, void* dst,
                                       int64_t bh, int64_t prefix_rows, int64_t suffix_rows, int64_t row_bytes,
                                       hipStream_t stream) {
  SPR_REQUIRE(prefix_rows >= 0 && suffix_rows >= 0, "spr_permute_concat_rows: negative size");
  SPR_REQUIRE(suffix_rows == 0 || suffix != nullptr, "spr_permute_concat_rows: null suffix");
  const int64_t rows = prefix_rows + suffix_rows;
  return launch_permute<MODE_CONCAT>(prefix, suffix, idx, dst, bh, rows, rows, prefix_rows, row_bytes, stream,
                                     "spr_permute_concat_rows");
}

// dst[b, j, :] = src[b, idx[b, j], :] for j < dst_rows (rows of src outside the
// index list are not read; out-of-range indices give zero rows).
extern "C" int spr_gather_rows(const void* src, int64_t src_rows, const int32_t* idx, void* dst,
                               int64_t dst_rows, int64_t bh, int64_t row_bytes, hipStream_t stream) {
  return launch_permute<MODE_GATHER>(src, nullptr, idx, dst, bh, src_rows, dst_rows, 0, row_bytes, stream,
                                     "spr_gather_rows");
}

// dst[b, idx[b, j], :] = src[b, j, :] for j < src_rows (other dst rows untouched).
extern "C" int spr_scatter_rows(const void* src, int64_t src_rows, const int32_t* idx, void* dst,
                                int64_t dst_rows, int64_t bh, int64_t row_bytes, hipStream_t stream) {
  return launch_permute<MODE_SCATTER>(src, nullptr, idx, dst, bh, src_rows, dst_rows, 0, row_bytes, stream,
                                      "spr_scatter_rows");
}
