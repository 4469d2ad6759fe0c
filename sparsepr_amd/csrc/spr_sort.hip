// Stable argsort of small-range cluster labels (counting sort), per row.
//
// Produces the `sorted_indices = argsort(labels)` that every permute call site
// computes with torch.argsort (reference permute.py:154-157, n8_v6.py:905,
// hunyuanvideo.py:189, kmeans_utils.py:1676) and the per-cluster sizes and
// start offsets that the block-sparse attention schedule and the centroid
// update consume.  Within a cluster tokens keep ascending index order.
//
// Three launches, all HBM/latency-light:
//   1. per (row, chunk of CHUNK tokens) label histogram in LDS;
//   2. per row: label totals, exclusive scan over labels, per-chunk bases;
//   3. per (row, chunk): one wave walks the chunk in order, ranks equal labels
//      inside each 64-token group with readlane compares, scatters token ids.
// Labels outside [0, k) go to a trailing overflow bucket (sorted last).
#include "spr_common.h"

namespace {

constexpr int CHUNK = 1024;
constexpr int MAX_BINS = 8192;  // k + 1 <= MAX_BINS (32 KB of LDS counters)

__device__ __forceinline__ uint32_t bin_of(int32_t label, int32_t k) {
  return (label >= 0 && label < k) ? static_cast<uint32_t>(label) : static_cast<uint32_t>(k);
}

__global__ __launch_bounds__(256) void label_hist_kernel(const int32_t* __restrict__ labels, int64_t n,
                                                         int32_t k, int32_t nchunks,
                                                         int32_t* __restrict__ hist) {
  extern __shared__ int32_t h[];  // [k + 1]
  const int32_t bins = k + 1;
  const int64_t row = blockIdx.y;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * CHUNK;
  for (int j = threadIdx.x; j < bins; j += blockDim.x) h[j] = 0;
  __syncthreads();
  const int64_t c1 = c0 + CHUNK < n ? c0 + CHUNK : n;
  for (int64_t t = c0 + threadIdx.x; t < c1; t += blockDim.x) {
    atomicAdd(&h[bin_of(labels[row * n + t], k)], 1);
  }
  __syncthreads();
  int32_t* out = hist + (row * nchunks + blockIdx.x) * bins;
  for (int j = threadIdx.x; j < bins; j += blockDim.x) out[j] = h[j];
}

// One block per row.  hist[row][chunk][bin] counts -> bases (in place).
__global__ __launch_bounds__(1024) void label_scan_kernel(int32_t* __restrict__ hist, int32_t k,
                                                          int32_t nchunks, int32_t* __restrict__ sizes,
                                                          int32_t* __restrict__ offsets) {
  __shared__ int32_t tot[MAX_BINS];
  __shared__ int32_t wsum[16];
  constexpr int U = 8;  // chunk rows in flight per thread
  const int32_t bins = k + 1;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int32_t* hrow = hist + row * static_cast<int64_t>(nchunks) * bins;
  for (int j = tid; j < bins; j += blockDim.x) {
    int32_t s = 0;
    int c = 0;
    for (; c + U <= nchunks; c += U) {
      int32_t v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = hrow[(c + u) * bins + j];
#pragma unroll
      for (int u = 0; u < U; ++u) s += v[u];
    }
    for (; c < nchunks; ++c) s += hrow[c * bins + j];
    tot[j] = s;
  }
  __syncthreads();
  // exclusive scan of tot[0..bins): a contiguous segment per thread, segment sums
  // scanned across the block with wave shuffles
  const int per = (bins + blockDim.x - 1) / blockDim.x;
  const int lo = tid * per;
  const int hi = lo + per < bins ? lo + per : bins;
  int32_t seg = 0;
  for (int j = lo; j < hi; ++j) seg += tot[j];
  int32_t incl = seg;
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t up = __shfl_up(incl, o, 64);
    if (lane >= o) incl += up;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int32_t before = 0;
  for (int w = 0; w < wave; ++w) before += wsum[w];
  {
    int32_t run = before + incl - seg;
    for (int j = lo; j < hi; ++j) {
      int32_t v = tot[j];
      if (sizes != nullptr && j < k) sizes[row * k + j] = v;
      tot[j] = run;
      run += v;
    }
  }
  __syncthreads();
  for (int j = tid; j < bins; j += blockDim.x) {
    if (offsets != nullptr) offsets[row * (k + 1) + j] = tot[j];
    int32_t run = tot[j];
    int c = 0;
    for (; c + U <= nchunks; c += U) {
      int32_t v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = hrow[(c + u) * bins + j];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        hrow[(c + u) * bins + j] = run;
        run += v[u];
      }
    }
    for (; c < nchunks; ++c) {
      int32_t a = hrow[c * bins + j];
      hrow[c * bins + j] = run;
      run += a;
    }
  }
}

// One wave per (row, chunk): ranks must follow token order, so the chunk is
// walked in 64-token groups by a single wave.
__global__ __launch_bounds__(64) void label_scatter_kernel(const int32_t* __restrict__ labels, int64_t n,
                                                           int32_t k, int32_t nchunks,
                                                           const int32_t* __restrict__ bases,
                                                           int32_t* __restrict__ sorted_idx) {
  extern __shared__ int32_t cnt[];  // [k + 1]
  const int32_t bins = k + 1;
  const int nbits = 32 - __builtin_clz(static_cast<uint32_t>(bins));  // 2^nbits > k + 1 > every bin
  const int64_t row = blockIdx.y;
  const int lane = threadIdx.x;
  const int32_t* b = bases + (row * nchunks + blockIdx.x) * bins;
  for (int j = lane; j < bins; j += 64) cnt[j] = b[j];
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * CHUNK;
  const int64_t c1 = c0 + CHUNK < n ? c0 + CHUNK : n;
  // all of the chunk's labels are loaded before the first ranking step
  constexpr int GROUPS = CHUNK / 64;
  int32_t bins_of[GROUPS];
#pragma unroll
  for (int i = 0; i < GROUPS; ++i) {
    const int64_t t = c0 + i * 64 + lane;
    bins_of[i] = t < c1 ? static_cast<int32_t>(bin_of(labels[row * n + t], k)) : -1;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < GROUPS; ++i) {
    const int64_t g = c0 + i * 64;
    if (g >= c1) break;
    const int64_t t = g + lane;
    const bool live = t < c1;
    const int32_t bin = bins_of[i];
    // lanes holding the same bin, one ballot per bin bit (nbits bits hold every bin and
    // keep the pattern of -1, past the chunk, apart from all of them); the rank is the
    // number of such lanes below this one, which keeps the sort stable
    uint64_t same = ~0ull;
    for (int bit = 0; bit < nbits; ++bit) {
      const bool set = (bin >> bit) & 1;
      const uint64_t m = __ballot(set);
      same &= set ? m : ~m;
    }
    const int rank = __popcll(same & ((1ull << lane) - 1ull));
    const int count = __popcll(same);
    int32_t pos = 0;
    if (live) pos = cnt[bin] + rank;
    __builtin_amdgcn_wave_barrier();
    if (live) {
      if (pos >= 0 && pos < n) sorted_idx[row * n + pos] = static_cast<int32_t>(t);
      if (rank == count - 1) cnt[bin] += count;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t count, int32_t value) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = value;
}

}  // namespace

extern "C" size_t spr_argsort_labels_workspace(int64_t rows, int64_t n, int32_t k) {
  const int64_t nchunks = spr::ceil_div(n, CHUNK);
  return static_cast<size_t>(rows * nchunks * (static_cast<int64_t>(k) + 1) * 4);
}

// labels int32 [rows, n] in [0, k) -> sorted_idx int32 [rows, n] (stable),
// sizes int32 [rows, k] (nullable), offsets int32 [rows, k + 1] (nullable).
extern "C" int spr_argsort_labels(const int32_t* labels, int64_t rows, int64_t n, int32_t k,
                                  int32_t* sorted_idx, int32_t* sizes, int32_t* offsets, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  SPR_REQUIRE(rows >= 0 && n >= 0, "spr_argsort_labels: negative size");
  SPR_REQUIRE(k >= 1 && k + 1 <= MAX_BINS, "spr_argsort_labels: k=%d outside [1, %d]", k, MAX_BINS - 1);
  SPR_REQUIRE(n < (int64_t(1) << 31), "spr_argsort_labels: n too large");
  SPR_REQUIRE(rows <= 65535, "spr_argsort_labels: rows=%lld exceeds 65535", (long long)rows);
  if (rows == 0) return SPR_OK;
  if (n == 0) {
    // Empty rows: sizes and offsets are all zero.
    if (sizes) fill_i32_kernel<<<64, 256, 0, stream>>>(sizes, rows * k, 0);
    if (offsets) fill_i32_kernel<<<64, 256, 0, stream>>>(offsets, rows * (k + 1), 0);
    SPR_LAUNCHED("spr_argsort_labels");
    return SPR_OK;
  }
  SPR_REQUIRE(labels && sorted_idx && workspace, "spr_argsort_labels: null pointer");
  const size_t need = spr_argsort_labels_workspace(rows, n, k);
  if (workspace_bytes < need) {
    spr_set_error("spr_argsort_labels: workspace %zu < %zu bytes", workspace_bytes, need);
    return SPR_EWORKSPACE;
  }
  const int32_t nchunks = static_cast<int32_t>(spr::ceil_div(n, CHUNK));
  int32_t* hist = static_cast<int32_t*>(workspace);
  const size_t bin_bytes = static_cast<size_t>(k + 1) * sizeof(int32_t);
  label_hist_kernel<<<dim3(nchunks, rows), 256, bin_bytes, stream>>>(labels, n, k, nchunks, hist);
  SPR_LAUNCHED("label_hist_kernel");
  label_scan_kernel<<<dim3(rows), 1024, 0, stream>>>(hist, k, nchunks, sizes, offsets);
  SPR_LAUNCHED("label_scan_kernel");
  label_scatter_kernel<<<dim3(nchunks, rows), 64, bin_bytes, stream>>>(labels, n, k, nchunks, hist, sorted_idx);
  SPR_LAUNCHED("label_scatter_kernel");
  return SPR_OK;
}
