// Block-sparse attention over cluster-pair blocks, and split-key dense attention
// for probe queries (v_mfma_f32_32x32x16_bf16, fp32 online softmax).
//
// Replaces:
//   dynamic_block_sparse_fwd_flashinfer -> FlashInfer VariableBlockSparseAttentionWrapper
//       (src/sparsepr/kmeans_utils.py:2164-2350); semantics of dynamic_block_sparse_fwd_torch
//       (kmeans_utils.py:1748-1841)
//   dense probe attention F.scaled_dot_product_attention (src/sparsepr/models/common/n8_v6.py:1236-1243)
//
// Layout: Q [BHq, S, D], K/V [BHkv, S, D] bf16 rows, cluster-contiguous (the
// permuted layout).  A query row of q-cluster a attends every key of every
// k-cluster c with map[a, c]; empty rows output 0 (lse -inf).
//
// Plan (one workgroup per kv head): cluster offsets, 128- and 256-row tiles per
// q-cluster, and for every q-cluster the ascending list of kept non-empty
// k-cluster key ranges ("segments").  The attention kernels walk a q-cluster's
// segments as one virtual key sequence in 64-key chunks, so cluster tails cost
// no MFMA work.
//
// Every wave owns 32 query rows of one q-cluster:
//   S^T[key, q] = K Q^T : A = 32 keys x 16 dims from the K tile in LDS, B = the
//                         wave's 32 query rows (registers, loaded once).
//   O^T[d, q]  += V^T P^T: A = 32 dims x 16 keys of V^T from LDS, B = P straight
//                         from the S^T accumulator (bf16), so a lane owns one
//                         query row for S, P and O: the row max/sum needs one
//                         exchange with lane l ^ 32 and nothing else.
// The key order inside a 16-key MFMA step is permuted consistently in P and V
// (key(t, h, e) = 16t + 8(e/4) + 4h + e%4), which makes P a plain slice of the
// accumulator.
//
// Kernels: attn_pipe_kernel (D = 128 block-sparse: 256-row tiles, K/V DMA'd
// into swizzled LDS tiles, next-S/softmax pipelining) and attn_fwd_kernel
// (D = 64 block-sparse and the dense probe attention: 128-row tiles, K/V
// staged through registers into a padded K tile and a transposed V tile,
// double-buffered, the next chunk fetched while the current one computes).
#include "spr_common.h"
#include <mutex>
#include <type_traits>

namespace {

using spr::u32x4;

constexpr int BM = 128;       // query rows per workgroup
constexpr int BN = 64;        // keys per chunk
constexpr int THREADS = 256;  // 4 waves

// A kept key range as seen by the virtual key sequence of one q-cluster: virtual
// positions [previous vend, vend) map to key rows delta + position.
struct Seg {
  int32_t delta;
  int32_t vend;
};

constexpr int MAX_LDS_SEGS = 768;  // segment lists up to this length are staged in LDS
#ifndef ATTN_NW
#define ATTN_NW 4  // block-sparse kernel: waves per workgroup
#define ATTN_QB 1  //                      32-row query blocks per wave
#endif

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// The element type of Q, K, V, P and the output: bf16 (F16 false) or fp16 (F16 true).  The
// MFMA, the packing of two fp32 values (round to nearest even) and the row sum of two
// packed probabilities (v_dot2_f32_bf16 / v_dot2_f32_f16) follow it.
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
template <bool F16>
__device__ __forceinline__ spr::f32x16 mfma16(u32x4 a, u32x4 b, spr::f32x16 c) {
  if constexpr (F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(a), spr::as_bf16x8(b), c, 0, 0, 0);
  }
}
template <bool F16>
__device__ __forceinline__ uint32_t pack2t(float lo, float hi) {
  if constexpr (F16) {
    const f16x2_t v = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    return pack2(lo, hi);
  }
}
// acc + lo + hi of a packed pair
template <bool F16>
__device__ __forceinline__ float dot2_ones(uint32_t pk, float acc) {
  if constexpr (F16) {
    const f16x2_t ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, pk), ones, acc, false);
  } else {
    const bf16x2_t ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk), ones, acc, false);
  }
}
// two NaNs of the element type
template <bool F16>
constexpr uint32_t nan_pair() {
  return F16 ? 0x7E007E00u : 0x7FC07FC0u;
}

// max / sum of x over lanes l and l ^ 32 (v_permlane32_swap exchanges the upper
// half-wave of one operand with the lower half of the other, so the two results
// hold x[l] and x[l ^ 32] in some order; max and + are symmetric in them).
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// max_xor32(x) * s for s > 0, as max(r0 * s, r1 * s): the products are canonical floats,
// so the max needs no canonicalising ops on the lane-swapped bits (one VALU op fewer).
__device__ __forceinline__ float max_xor32_scaled(float x, float s) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]) * s, __uint_as_float(r[1]) * s);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Column of chunk key p in a V^T row: bits 2 and 3 of p swapped, so the keys
// 16t + 4h + {0..3} and 16t + 8 + 4h + {0..3} of one MFMA A fragment (lane half
// h, k-step t) sit in the 8 consecutive columns 16t + 8h + {0..7}.
__device__ __forceinline__ int v_col(int p) { return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1); }

// Threshold (log2 units) by which a row maximum must grow before the running
// output is rescaled; p = 2^(s - m) stays below 2^8 in between.
constexpr float RESCALE_SLACK = 8.0f;

// D = 16: one 32-dim block of O^T whose rows 16 .. 31 (V^T rows kept at zero) are not
// stored.  With fewer K pieces or V pairs per chunk than threads, the threads past them
// load and stash nothing.
template <int D, int NTHREADS>
struct Tile {
  static constexpr int KSTEPS = D / 16;
  static constexpr int DBLK = D >= 32 ? D / 32 : 1;
  static constexpr int VD = 32 * DBLK;       // dim rows of the V^T tile
  static constexpr int K_ROW = D * 2 + 16;   // bytes per key row of the K tile (+16 pad)
  static constexpr int V_ROW = BN * 2 + 16;  // bytes per dim row of the V^T tile (+16 pad: 8 consecutive
                                             // rows cover all 32 banks, so 128-bit reads are conflict-free)
  static constexpr int K_BYTES = BN * K_ROW;
  static constexpr int V_BYTES = VD * V_ROW;
  static constexpr int K_ITEMS = BN * D / 8;         // 16-byte K pieces per chunk
  static constexpr int V_ITEMS = (BN / 2) * (D / 8);  // (2 rows x 16 bytes) V pairs per chunk
  static constexpr int K_PIECES = (K_ITEMS + NTHREADS - 1) / NTHREADS;  // per thread
  static constexpr int V_PAIRS = (V_ITEMS + NTHREADS - 1) / NTHREADS;
  static_assert(D % 16 == 0 && D <= 128, "unsupported head dim");
};

// ---------------------------------------------------------------------------- plan

// Workspace layout per kv head (int32 units), see plan_words().
struct PlanView {
  int32_t* q_off;      // [Qc + 1]
  int32_t* tile_off;   // [Qc + 1] first BM-row tile of each q-cluster
  int32_t* tile2_off;  // [Qc + 1] first 2*BM-row tile of each q-cluster
  int32_t* nseg;       // [Qc]
  int32_t* total;     // [Qc]
  Seg* segs;          // [Qc][Kc]
  int32_t* qc_by_len;     // [Qc] q-clusters by decreasing key count (ties by index)
  int32_t* tile2_sorted;  // [Qc + 1] first 2*BM-row tile of each in that order
};

// Word offset of a head's segment list, rounded up to even so that (with an even
// plan_words) every head's Seg array is 8-byte aligned.
__host__ __device__ inline int64_t plan_seg_offset(int32_t qn) { return (5 * (int64_t)qn + 3 + 1) & ~int64_t(1); }

__host__ __device__ inline int64_t plan_words(int32_t qn, int32_t kn) {
  // q_off, tile_off, tile2_off [qn + 1] each, nseg, total [qn] each, (pad), segs [qn][kn]
  // pairs, qc_by_len [qn], tile2_sorted [qn + 1], then a pad word: an even count
  return plan_seg_offset(qn) + 2 * (int64_t)qn * kn + 2 * (int64_t)qn + 2;
}

// After the bh_kv per-head plans: head_order[bh_kv], the kv head processed in each kv-head
// slot of the 256-row tile grid (see attn_head_order_kernel), then the plan header.
__host__ __device__ inline int32_t* head_order_at(int32_t* base, int64_t bh_kv, int32_t qn, int32_t kn) {
  return base + bh_kv * plan_words(qn, kn);
}

// Plan header (5 words after head_order): magic, bh_kv, qn, kn, s.  The plan kernels
// write it last; the attention kernels compare it with their own arguments and do
// nothing when it does not match, so a plan built for other sizes (or never built)
// cannot send them past the ends of the plan, Q or K/V.
constexpr int32_t PLAN_MAGIC = 0x50525053;  // "SPRP"
constexpr int PLAN_HEADER_WORDS = 5;
__host__ __device__ inline const int32_t* plan_header_at(const int32_t* base, int64_t bh_kv, int32_t qn, int32_t kn) {
  return base + bh_kv * plan_words(qn, kn) + bh_kv;
}
__device__ inline bool plan_matches(const int32_t* base, int64_t bh_kv, int32_t qn, int32_t kn, int32_t s) {
  const int32_t* hd = plan_header_at(base, bh_kv, qn, kn);
  return hd[0] == PLAN_MAGIC && hd[1] == static_cast<int32_t>(bh_kv) && hd[2] == qn && hd[3] == kn && hd[4] == s;
}

// A plan built for other sizes: the whole (1-D) grid writes NaN over the output [bh_q, s, d]
// bf16 and the LSE [bh_q, s] (when given), each workgroup a strided share, so the caller sees
// the mismatch instead of stale memory.  d is 64 or 128, so the output is whole 16-byte pieces.
__device__ inline void fill_nan_output(uint16_t* out, float* lse, int64_t bh_q, int32_t s, int32_t d, uint32_t nan2) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t pieces = bh_q * s * (d / 8);
  const spr::u32x4 nan8 = {nan2, nan2, nan2, nan2};
  for (int64_t i = first; i < pieces; i += step) reinterpret_cast<spr::u32x4*>(out)[i] = nan8;
  if (lse != nullptr) {
    for (int64_t i = first; i < bh_q * s; i += step) lse[i] = __builtin_nanf("");
  }
}

__host__ __device__ inline PlanView plan_at(int32_t* base, int64_t h, int32_t qn, int32_t kn) {
  int32_t* p = base + h * plan_words(qn, kn);
  PlanView v;
  v.q_off = p;
  v.tile_off = p + (qn + 1);
  v.tile2_off = p + 2 * (qn + 1);
  v.nseg = p + 3 * (qn + 1);
  v.total = v.nseg + qn;
  v.segs = reinterpret_cast<Seg*>(p + plan_seg_offset(qn));
  v.qc_by_len = p + plan_seg_offset(qn) + 2 * (int64_t)qn * kn;
  v.tile2_sorted = v.qc_by_len + qn;
  return v;
}

// The kept k-clusters of a q-cluster row come from the map (map != nullptr) or from a
// selector schedule: ids [bh, qn, kn] int32 with counts [bh, qn] (the ascending kept ids
// svg_ear_select_budget_schedule / compact_selected_clusters emit, n8_ops.cu:573-638).  A
// schedule entry outside [0, kn) or not above the entry before it is ignored, so every
// key range enters a row's segment list at most once, in ascending order: the plan is
// the same as from the equivalent map.
__global__ __launch_bounds__(THREADS) void attn_plan_kernel(const uint8_t* __restrict__ map,
                                                            const int32_t* __restrict__ ids,
                                                            const int32_t* __restrict__ counts,
                                                            const int32_t* __restrict__ q_sizes,
                                                            const int32_t* __restrict__ k_sizes, int32_t qn,
                                                            int32_t kn, int32_t s_rows, int32_t* __restrict__ plan) {
  extern __shared__ int32_t k_off[];  // [kn + 1]
  const int64_t h = blockIdx.x;
  PlanView pv = plan_at(plan, h, qn, kn);
  const int32_t* qs = q_sizes + h * qn;
  const int32_t* ks = k_sizes + h * kn;
  // Offsets are running sums clamped at s_rows; the sizes are clamped at zero, so the
  // clamped running sum equals min(prefix sum, s_rows) and wave scans compute it.
  const int wv = threadIdx.x >> 6;
  const int ln = threadIdx.x & 63;
  auto scan64 = [&](int64_t v) {  // inclusive scan over the wave
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t up = __shfl_up(v, o, 64);
      if (ln >= o) v += up;
    }
    return v;
  };
  if (wv == 0) {  // k-cluster offsets (every workgroup of the head, for its rows)
    int64_t carry = 0;
    for (int c0 = 0; c0 < kn; c0 += 64) {
      const int c = c0 + ln;
      const int64_t own = c < kn ? max(ks[c], 0) : 0;
      const int64_t incl = scan64(own);
      if (c < kn) k_off[c] = static_cast<int32_t>(min(carry + incl - own, static_cast<int64_t>(s_rows)));
      carry += __shfl(incl, 63, 64);
    }
    if (ln == 0) k_off[kn] = static_cast<int32_t>(min(carry, static_cast<int64_t>(s_rows)));
  } else if (wv == 1 && blockIdx.y == 0) {  // q-cluster offsets and tile counts
    int64_t carry = 0, tcarry = 0, t2carry = 0;
    for (int i0 = 0; i0 < qn; i0 += 64) {
      const int i = i0 + ln;
      const int64_t own = i < qn ? max(qs[i], 0) : 0;
      const int64_t incl = scan64(own);
      const int64_t qrun = min(carry + incl - own, static_cast<int64_t>(s_rows));
      const int64_t next = min(carry + incl, static_cast<int64_t>(s_rows));
      const int64_t tl = i < qn ? (next - qrun + BM - 1) / BM : 0;
      const int64_t tl2 = i < qn ? (next - qrun + 2 * BM - 1) / (2 * BM) : 0;
      const int64_t ti = scan64(tl), ti2 = scan64(tl2);
      if (i < qn) {
        pv.q_off[i] = static_cast<int32_t>(qrun);
        pv.tile_off[i] = static_cast<int32_t>(tcarry + ti - tl);
        pv.tile2_off[i] = static_cast<int32_t>(t2carry + ti2 - tl2);
      }
      carry += __shfl(incl, 63, 64);
      tcarry += __shfl(ti, 63, 64);
      t2carry += __shfl(ti2, 63, 64);
    }
    if (ln == 0) {
      pv.q_off[qn] = static_cast<int32_t>(min(carry, static_cast<int64_t>(s_rows)));
      pv.tile_off[qn] = static_cast<int32_t>(tcarry);
      pv.tile2_off[qn] = static_cast<int32_t>(t2carry);
    }
  }
  __syncthreads();
  // one wave per q-cluster row: ascending compaction of kept, non-empty k-clusters
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  for (int i = blockIdx.y * (THREADS / 64) + wave; i < qn; i += gridDim.y * (THREADS / 64)) {
    const int64_t row = h * qn + i;
    Seg* out = pv.segs + static_cast<int64_t>(i) * kn;
    int32_t count = 0;
    int32_t total = 0;
    // map: walk the kn flags; schedule: walk the row's min(count, kn) ids
    const int32_t n_in = map != nullptr ? kn : min(max(counts[row], 0), kn);
    int32_t last = -1;  // schedule: the last id taken so far
    for (int c0 = 0; c0 < n_in; c0 += 64) {
      int c;
      bool listed;
      if (map != nullptr) {
        c = c0 + lane;
        listed = c < kn && map[row * kn + c] != 0;
      } else {
        // taken iff in range and above every earlier id of the row (a max-scan)
        c = c0 + lane < n_in ? ids[row * kn + c0 + lane] : -1;
        int run = c;
        for (int o = 1; o < 64; o <<= 1) {
          const int up = __shfl_up(run, o, 64);
          if (lane >= o) run = max(run, up);
        }
        int before = __shfl_up(run, 1, 64);
        before = max(lane == 0 ? -1 : before, last);
        listed = c0 + lane < n_in && c >= 0 && c < kn && c > before;
        last = max(last, __shfl(run, 63, 64));
      }
      int32_t len = 0, start = 0;
      if (listed) {
        start = k_off[c];
        len = k_off[c + 1] - start;
      }
      const bool keep = listed && len > 0;
      const uint64_t bits = __ballot(keep);
      const int pos = __popcll(bits & ((1ull << lane) - 1ull));
      int32_t incl = keep ? len : 0;  // inclusive scan of kept lengths over the wave
      for (int o = 1; o < 64; o <<= 1) {
        const int32_t up = __shfl_up(incl, o, 64);
        if (lane >= o) incl += up;
      }
      const int32_t vend = total + incl;
      if (keep) out[count + pos] = Seg{start - (vend - len), vend};
      total += __shfl(incl, 63, 64);
      count += __popcll(bits);
    }
    if (lane == 0) {
      pv.nseg[i] = count;
      pv.total[i] = total;
    }
  }
}

// ---------------------------------------------------------------------------- main kernel

// MODE 0: block-sparse (plan), output normalised bf16 + optional lse.
//         1-D grid; workgroup b runs on XCD b % 8 and takes logical tile
//         (b % 8) * (gridDim.x / 8) + b / 8, so consecutive tiles (the tiles of
//         one q-cluster, which read the same key blocks) share one XCD's L2.
// MODE 1: dense split-key for probe rows: q rows [0, m) of a [BHq, m, D] tensor,
//         keys [split * split_len, ...) of K/V; output unnormalised fp32 partials.
// NW waves per workgroup, QB 32-row query blocks per wave (NW * QB * 32 = BM).
// KIDX: keys are gathered through k_index (a compile-time switch, so the plain
// path carries no global load, and no wait on one, in its chunk planning).
// QB = 2 runs one wave per SIMD with the output accumulators in AGPRs: every K
// and V fragment read from LDS then feeds two MFMAs, and each wave carries twice
// as many independent MFMA chains.
template <int D, int MODE, bool SEGL, int NW, int QB, bool KIDX, bool F16>
__global__ __launch_bounds__(NW * 64, QB == 2 ? 1 : 2) void attn_fwd_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    int32_t s_q, int32_t s_kv, int32_t group, int32_t qn, int32_t kn, const int32_t* __restrict__ plan,
    int32_t bh_q, int32_t tiles_per_head, float scale_log2, const int32_t* __restrict__ q_index,
    const int32_t* __restrict__ k_index, uint16_t* __restrict__ out, float* __restrict__ lse, int32_t split_len, float* __restrict__ part_o,
    float* __restrict__ part_ml, int64_t kv_stride) {
  // kv_stride: elements from one kv head's rows to the next (s_kv * D when packed)
  constexpr int NT = NW * 64;
  static_assert(NW * QB * 32 == BM, "tile shape");
  using T = Tile<D, NT>;
  __shared__ __attribute__((aligned(16))) uint8_t k_tile[2][T::K_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t v_tile[2][T::V_BYTES];
  __shared__ int32_t key_rows[4][BN];
  __shared__ Seg seg_lds[SEGL ? MAX_LDS_SEGS : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;

  // ---- work item
  int64_t bhq;
  int32_t row0, row1;        // query rows of this tile: [row0, row1)
  const Seg* segs = nullptr;  // global copy of the segment list (MODE 0)
  int32_t nseg = 0;
  int32_t total;
  int32_t dense_k0 = 0;
  if constexpr (MODE == 0) {
    const int64_t per_xcd = gridDim.x / 8;
    const int64_t logical = static_cast<int64_t>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    bhq = logical / tiles_per_head;
    const int32_t t = static_cast<int32_t>(logical - bhq * tiles_per_head);
    if (!plan_matches(plan, bh_q / group, qn, kn, s_q)) {
      fill_nan_output(out, lse, bh_q, s_q, D, nan_pair<F16>());
      return;
    }
    if (bhq >= bh_q) return;
    PlanView pv = plan_at(const_cast<int32_t*>(plan), bhq / group, qn, kn);
    if (t >= pv.tile_off[qn]) return;
    int lo = 0, hi = qn;  // largest i with tile_off[i] <= t
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (pv.tile_off[mid] <= t) lo = mid; else hi = mid;
    }
    const int qc = lo;
    row0 = pv.q_off[qc] + (t - pv.tile_off[qc]) * BM;
    row1 = min(row0 + BM, pv.q_off[qc + 1]);
    segs = pv.segs + static_cast<int64_t>(qc) * kn;
    nseg = pv.nseg[qc];
    total = pv.total[qc];
  } else {
    bhq = blockIdx.z;
    row0 = blockIdx.y * BM;
    row1 = min(row0 + BM, s_q);
    dense_k0 = blockIdx.x * split_len;
    const int32_t k1 = min(dense_k0 + split_len, s_kv);
    total = max(k1 - dense_k0, 0);
  }
  const int64_t bhkv = bhq / group;

  const uint16_t* qb = q + bhq * static_cast<int64_t>(s_q) * D;
  const uint16_t* kb = k + bhkv * kv_stride;
  const uint16_t* vb = v + bhkv * kv_stride;
  // raw buffer views of this head's K and V: 32-bit offsets, reads past the end return 0
  const int32_t kv_bytes = s_kv * D * 2;
  const __amdgpu_buffer_rsrc_t k_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kb), 0, kv_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vb), 0, kv_bytes, 0x00020000);
  if constexpr (MODE == 0 && SEGL) {
    for (int i = tid; i < nseg; i += NT) seg_lds[i] = segs[i];
  }

  // ---- this lane's query rows (one per block), as MFMA B fragments over the head dim.
  // With q_index, tile row r is the query stored at row q_index[r] (the layout of
  // q, out and lse); rows outside [0, s_q) are treated as absent.
  int32_t my_row[QB];
  bool row_live[QB];
  u32x4 qf[QB][T::KSTEPS];
#pragma unroll
  for (int j = 0; j < QB; ++j) {
    my_row[j] = row0 + (wave * QB + j) * 32 + col;
    row_live[j] = my_row[j] < row1;
    if (q_index != nullptr && row_live[j]) {
      my_row[j] = q_index[bhq * static_cast<int64_t>(s_q) + my_row[j]];
      row_live[j] = my_row[j] >= 0 && my_row[j] < s_q;
    }
#pragma unroll
    for (int s = 0; s < T::KSTEPS; ++s) {
      qf[j][s] = row_live[j]
                     ? *reinterpret_cast<const u32x4*>(qb + static_cast<int64_t>(my_row[j]) * D + s * 16 + half * 8)
                     : u32x4{0, 0, 0, 0};
    }
  }

  spr::f32x16 o_acc[QB][T::DBLK];
  float m_run[QB], l_run[QB];  // running max (log2 units, may lag the true max by < RESCALE_SLACK), sum
#pragma unroll
  for (int j = 0; j < QB; ++j) {
#pragma unroll
    for (int b = 0; b < T::DBLK; ++b) o_acc[j][b] = spr::f32x16{};
    m_run[j] = -__builtin_huge_valf();
    l_run[j] = 0.0f;
  }

  const int nch = (total + BN - 1) / BN;

  // Wave 0 writes the key row of every position of a chunk three chunks ahead
  // (ring of 4); every thread reads the rows it loads one chunk before it loads
  // them, so global loads issue without waiting on LDS.  Positions past the end
  // repeat the last key (their scores are masked), so every load is unconditional.
  int32_t cur_s = 0;  // segment holding the first position of the next chunk to plan
  auto seg_of = [&](int32_t vpos) {
    int32_t s = cur_s;
    if constexpr (SEGL) {
      while (s < nseg - 1 && vpos >= seg_lds[s].vend) ++s;
    } else {
      while (s < nseg - 1 && vpos >= segs[s].vend) ++s;
    }
    return s;
  };
  auto plan_chunk = [&](int c) {
    if (wave == 0) {
      const int32_t vpos = min(c * BN + lane, total - 1);
      if constexpr (MODE == 0) {
        const int32_t s = seg_of(vpos);
        int32_t delta;
        if constexpr (SEGL) delta = seg_lds[s].delta; else delta = segs[s].delta;
        // with k_index, cluster-sorted key position p is stored at row k_index[p]
        // (a bad index only reads zeros: the K/V loads are range-checked)
        if constexpr (KIDX) {
          key_rows[c % 4][lane] = k_index[bhkv * static_cast<int64_t>(s_kv) + delta + vpos];
        } else {
          key_rows[c % 4][lane] = delta + vpos;
        }
        cur_s = __builtin_amdgcn_readlane(s, 63);
      } else {
        key_rows[c % 4][lane] = dense_k0 + vpos;
      }
    }
  };

  u32x4 kreg[T::K_PIECES];
  u32x4 vreg[T::V_PAIRS][2];
  auto bload = [](__amdgpu_buffer_rsrc_t r, int32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  };
  int32_t krow[T::K_PIECES];  // key rows of this thread's K pieces in the next chunk to fetch
  int32_t vrow[2];              // key rows of this thread's two V rows
  // K piece i of this thread: item tid + i NT (valid below K_ITEMS) is row item / (D / 8),
  // piece item % (D / 8); V pair i: item tid + i NT (valid below V_ITEMS) is rows 2 rp,
  // 2 rp + 1 (rp = tid % 32, the same for every i) and piece item / 32
  auto k_live = [&](int i) { return tid + i * NT < T::K_ITEMS; };
  auto v_live = [&](int i) { return tid + i * NT < T::V_ITEMS; };
  auto load_rows = [&](int c) {  // plain copies, so nothing waits on these reads until fetch()
    const int32_t* kr = key_rows[c % 4];
#pragma unroll
    for (int i = 0; i < T::K_PIECES; ++i) krow[i] = k_live(i) ? kr[(tid + i * NT) / (D / 8)] : 0;
    const int rp = tid % (BN / 2);
    vrow[0] = kr[2 * rp];
    vrow[1] = kr[2 * rp + 1];
  };
  auto fetch_k = [&]() {
#pragma unroll
    for (int i = 0; i < T::K_PIECES; ++i) kreg[i] = bload(k_rsrc, krow[i] * (D * 2) + (tid % (D / 8)) * 16);
  };
  auto fetch_v = [&]() {
#pragma unroll
    for (int i = 0; i < T::V_PAIRS; ++i) {
      const int pc = v_live(i) ? (tid + i * NT) / (BN / 2) : 0;
      vreg[i][0] = bload(v_rsrc, vrow[0] * (D * 2) + pc * 16);
      vreg[i][1] = bload(v_rsrc, vrow[1] * (D * 2) + pc * 16);
    }
  };
  auto stash_k = [&](int buf) {
#pragma unroll
    for (int i = 0; i < T::K_PIECES; ++i) {
      if (!k_live(i)) continue;
      const int r = (tid + i * NT) / (D / 8);
      const int pc = tid % (D / 8);
      *reinterpret_cast<u32x4*>(&k_tile[buf][r * T::K_ROW + pc * 16]) = kreg[i];
    }
  };
  auto stash_v = [&](int buf) {
    const int rp = tid % (BN / 2);
    const int vc = v_col(2 * rp);  // keys 2rp, 2rp + 1 land in columns vc, vc + 1
#pragma unroll
    for (int i = 0; i < T::V_PAIRS; ++i) {
      if (!v_live(i)) continue;
      const int pc = (tid + i * NT) / (BN / 2);
      const uint32_t a[4] = {vreg[i][0].x, vreg[i][0].y, vreg[i][0].z, vreg[i][0].w};
      const uint32_t b[4] = {vreg[i][1].x, vreg[i][1].y, vreg[i][1].z, vreg[i][1].w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        // dims pc*8 + 2w (low halves of a, b) and pc*8 + 2w + 1 (high halves)
        const uint32_t lo = __builtin_amdgcn_perm(b[w], a[w], 0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(b[w], a[w], 0x07060302u);
        *reinterpret_cast<uint32_t*>(&v_tile[buf][(pc * 8 + 2 * w) * T::V_ROW + vc * 2]) = lo;
        *reinterpret_cast<uint32_t*>(&v_tile[buf][(pc * 8 + 2 * w + 1) * T::V_ROW + vc * 2]) = hi;
      }
    }
  };

  if constexpr (T::VD > D) {  // V^T rows past the head dim stay zero in both buffers
    for (int e = tid; e < 2 * (T::VD - D) * (T::V_ROW / 4); e += NT) {
      const int b = e / ((T::VD - D) * (T::V_ROW / 4)), w = e % ((T::VD - D) * (T::V_ROW / 4));
      reinterpret_cast<uint32_t*>(&v_tile[b][D * T::V_ROW])[w] = 0u;
    }
  }
  if (nch > 0) {
    if constexpr (MODE == 0 && SEGL) __syncthreads();  // staged segment list visible to wave 0
    plan_chunk(0);
    if (nch > 1) plan_chunk(1);
    if (nch > 2) plan_chunk(2);
    __syncthreads();
    load_rows(0);
    fetch_k();
    fetch_v();
    if (nch > 1) load_rows(1);
    stash_k(0);
    stash_v(0);
    __syncthreads();
  }

  // Complete the query loads here, on every path into the loop, so that no wait
  // for them is left to the loop body (where it would also drain the loads of
  // the next chunk, which share the in-order counter).
#pragma unroll
  for (int j = 0; j < QB; ++j) {
#pragma unroll
    for (int s = 0; s < T::KSTEPS; ++s) asm volatile("" ::"v"(qf[j][s].x), "v"(qf[j][s].y), "v"(qf[j][s].z), "v"(qf[j][s].w));
  }
  // Per chunk: K of chunk c + 1 is fetched at the top and stashed after the
  // first 32-key half (its LDS buffer is free since the last barrier), then V of
  // chunk c + 1 is fetched and stashed at the end, so the two staging sets are
  // never live together.  Each half: S^T = K Q^T (each K fragment feeds the QB
  // query blocks of the wave), online softmax (log2 domain; a lane owns one
  // query row per block), O^T += V^T P^T.
  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    const bool more = c + 1 < nch;
    if (more) fetch_k();  // rows of chunk c + 1, read during chunk c - 1
    const int32_t left = total - c * BN;  // keys past the end exist only in the last chunk
#pragma unroll
    for (int kbk = 0; kbk < 2; ++kbk) {
      spr::f32x16 s_acc[QB];
#pragma unroll
      for (int j = 0; j < QB; ++j) s_acc[j] = spr::f32x16{};
      {
        const uint8_t* arow = &k_tile[buf][(kbk * 32 + col) * T::K_ROW + half * 16];
#pragma unroll
        for (int s = 0; s < T::KSTEPS; ++s) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(arow + s * 32);
#pragma unroll
          for (int j = 0; j < QB; ++j) {
            s_acc[j] = mfma16<F16>(a, qf[j][s], s_acc[j]);
          }
        }
      }
      if (kbk == 0 && c + 3 < nch) plan_chunk(c + 3);
      if (left < BN) {
#pragma unroll
        for (int j = 0; j < QB; ++j) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = kbk * 32 + 8 * (e / 4) + 4 * half + (e % 4);
            if (key >= left) s_acc[j][e] = -__builtin_huge_valf();
          }
        }
      }

      float mloc[QB];
      bool grow = false;
#pragma unroll
      for (int j = 0; j < QB; ++j) {
        float mx = -__builtin_huge_valf();
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s_acc[j][e]);
        mloc[j] = max_xor32_scaled(mx, scale_log2);
        grow = grow || (mloc[j] > m_run[j] + RESCALE_SLACK);
      }
      // Rescale lazily: only a row whose maximum grew by more than the slack moves its
      // running maximum, so a row's result does not depend on the other rows of its wave.
      if (__ballot(grow) != 0ull) {
#pragma unroll
        for (int j = 0; j < QB; ++j) {
          const bool up = mloc[j] > m_run[j] + RESCALE_SLACK;
          const float m_new = up ? mloc[j] : m_run[j];
          const float alpha = up ? __builtin_amdgcn_exp2f(m_run[j] - m_new) : 1.0f;
          l_run[j] *= alpha;
#pragma unroll
          for (int b = 0; b < T::DBLK; ++b) {
#pragma unroll
            for (int e = 0; e < 16; ++e) o_acc[j][b][e] *= alpha;
          }
          m_run[j] = m_new;
        }
      }
      uint32_t pf[QB][2][4];  // P of this half as bf16 pairs: [block][k-step][dword]
#pragma unroll
      for (int j = 0; j < QB; ++j) {
        const float neg_m = (m_run[j] == -__builtin_huge_valf()) ? 0.0f : -m_run[j];
        // The row sum adds the bf16-rounded probabilities that also weight V.
        float lsum0 = 0.0f, lsum1 = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_acc[j][e], scale_log2, neg_m));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_acc[j][e + 1], scale_log2, neg_m));
          const uint32_t pk = pack2t<F16>(p0, p1);
          pf[j][e / 8][(e % 8) / 2] = pk;
          if (e % 4 == 0) {
            lsum0 = dot2_ones<F16>(pk, lsum0);
          } else {
            lsum1 = dot2_ones<F16>(pk, lsum1);
          }
        }
        l_run[j] += lsum0 + lsum1;
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int t = kbk * 2 + tt;
#pragma unroll
        for (int b = 0; b < T::DBLK; ++b) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(&v_tile[buf][(b * 32 + col) * T::V_ROW + (16 * t + 8 * half) * 2]);
#pragma unroll
          for (int j = 0; j < QB; ++j) {
            const u32x4 bfrag = u32x4{pf[j][tt][0], pf[j][tt][1], pf[j][tt][2], pf[j][tt][3]};
            o_acc[j][b] = mfma16<F16>(a, bfrag, o_acc[j][b]);
          }
        }
      }
      if (kbk == 0 && more) {
        stash_k(buf ^ 1);
        fetch_v();
        if (c + 2 < nch) load_rows(c + 2);
      }
    }
    if (more) stash_v(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue
#pragma unroll
  for (int j = 0; j < QB; ++j) {
    const float l_tot = sum_xor32(l_run[j]);
    if constexpr (MODE == 0) {
      const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
      if (row_live[j]) {
        uint16_t* orow = out + (bhq * static_cast<int64_t>(s_q) + my_row[j]) * D;
#pragma unroll
        for (int b = 0; b < T::DBLK; ++b) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int d0 = b * 32 + 8 * i + 4 * half;
            if (d0 >= D) continue;  // D = 16: the block's upper 16 dims are padding
            uint2 w;
            w.x = pack2t<F16>(o_acc[j][b][4 * i] * inv, o_acc[j][b][4 * i + 1] * inv);
            w.y = pack2t<F16>(o_acc[j][b][4 * i + 2] * inv, o_acc[j][b][4 * i + 3] * inv);
            *reinterpret_cast<uint2*>(orow + d0) = w;
          }
        }
        if (lse != nullptr && half == 0) {
          lse[bhq * static_cast<int64_t>(s_q) + my_row[j]] =
              l_tot > 0.0f ? (m_run[j] + __builtin_amdgcn_logf(l_tot)) * 0.69314718055994531f
                           : -__builtin_huge_valf();
        }
      }
    } else {
      // partials: part_o [BHq, nsplit, s_q, D] fp32, part_ml [BHq, nsplit, s_q, 2]
      if (row_live[j]) {
        const int64_t slot = (bhq * gridDim.x + blockIdx.x) * static_cast<int64_t>(s_q) + my_row[j];
        float* po = part_o + slot * D;
#pragma unroll
        for (int b = 0; b < T::DBLK; ++b) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int d0 = b * 32 + 8 * i + 4 * half;
            if (d0 >= D) continue;
            *reinterpret_cast<spr::f32x4*>(po + d0) =
                spr::f32x4{o_acc[j][b][4 * i], o_acc[j][b][4 * i + 1], o_acc[j][b][4 * i + 2], o_acc[j][b][4 * i + 3]};
          }
        }
        if (half == 0) {
          part_ml[slot * 2] = m_run[j];
          part_ml[slot * 2 + 1] = l_tot;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------- block-sparse, D = 128: LDS layout
// K and V chunks are copied from HBM straight into LDS (buffer_load ... lds, 16
// bytes a lane, 1 KB per wave instruction): no staging registers and no staging
// work in the waves' instruction streams.
//
// Tiles hold 64 key rows of 256 bytes, row-major; the sixteen 16-byte pieces of
// row r are XOR-swizzled for the 64 four-byte LDS banks: piece j sits at slot
// j ^ (r & 15) in the K tile (the S^T A fragments, 128-bit reads of 16
// consecutive rows per cycle, cover all 64 banks) and at slot j ^ 4(r & 3) in
// the V tile.  V^T fragments come from the
// transposing read ds_read_b64_tr_b16: in each group of 16 lanes, output lane
// 4A + B receives element B of the 8-byte reads of lanes A, A + 4, A + 8 and
// A + 12.  Lane s of group g (A = s % 4, i = s / 4 within the group) therefore
// reads row 16t + 8r + 4h + i, dims 32b + 16(g & 1) + 4A, and output lane
// (dim d, half h) receives keys 16t + 8r + 4h + {0..3} of dim d: read r = 0, 1
// give the two 4-key halves of the A fragment in the key order the S^T
// accumulator produces (key(t, h, e) = 16t + 8(e/4) + 4h + e%4).  The 4 rows x
// 4 pieces each half-wave reads (pieces 4b .. 4b + 3) land in 16 distinct
// slots, all 64 banks.
constexpr int DROW = 256;         // bytes per key row (D = 128)
constexpr int DTILE = BN * DROW;  // bytes per K or V chunk tile

__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, int32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
#endif
}

struct alignas(8) u32x2 {
  uint32_t x, y;
};

__device__ __forceinline__ u32x2 lds_read_tr16(const uint8_t* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p)));
#else
  return u32x2{0, 0};
#endif
}

// ---------------------------------------------------------------------------- block-sparse, D = 128, pipelined
// The work items, plan walk and online softmax of attn_fwd_kernel MODE 0 over
// 256-row query tiles: eight waves of 32 rows (two per SIMD, one workgroup per
// CU) share each K/V chunk, which halves the HBM/L2 traffic and DMA issue per
// query row against 128-row tiles.  S^T of the next 32-key half is computed
// while the current half's probabilities are formed: after the row max and
// lazy rescale of half h, one straight-line block issues the MFMAs of S(h + 1),
// the exponentials of half h and the MFMAs of O += P(h) V, so the matrix unit
// works through the softmax.  Waves whose rows all lie past the tile's end keep
// the DMA and barriers and skip the compute.  S(h + 1) of a chunk's second half
// reads the next chunk's K tile, so the chunk barrier sits before that block
// and four LDS buffers rotate: chunk x is DMA'd right after the barrier of
// chunk x - 3 (its buffer's previous chunk, x - 4, was last read before it)
// and waited for before the barrier of chunk x - 1, two chunks later; key rows
// are planned four chunks ahead.
template <bool SEGL, bool KIDX, bool F16>
__global__ __launch_bounds__(512, 1) void attn_pipe_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int32_t s_q,
    int32_t s_kv, int32_t group, int32_t qn, int32_t kn, const int32_t* __restrict__ plan, int32_t bh_q,
    int32_t tiles_per_head, float scale_log2, const int32_t* __restrict__ q_index,
    const int32_t* __restrict__ k_index, uint16_t* __restrict__ out, float* __restrict__ lse) {
  constexpr int NW = 8;
  constexpr int D = 128;
  constexpr int KSTEPS = D / 16;
  constexpr int DBLK = D / 32;
  constexpr int NT = NW * 64;
  constexpr int TBM = NW * 32;
  constexpr int DMA_PER_WAVE = 16 / NW;
  __shared__ __attribute__((aligned(1024))) uint8_t k_tiles[4][DTILE];
  uint8_t* const k_tile0 = k_tiles[0];
  uint8_t* const k_tile1 = k_tiles[1];
  uint8_t* const k_tile2 = k_tiles[2];
  uint8_t* const k_tile3 = k_tiles[3];
  __shared__ __attribute__((aligned(1024))) uint8_t v_tiles[4][DTILE];
  uint8_t* const v_tile0 = v_tiles[0];
  uint8_t* const v_tile1 = v_tiles[1];
  uint8_t* const v_tile2 = v_tiles[2];
  uint8_t* const v_tile3 = v_tiles[3];
  __shared__ int32_t key_rows[4][BN];
  __shared__ Seg seg_lds[SEGL ? MAX_LDS_SEGS : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;

  // ---- work item: XCD-grouped order over 256-row tiles; head slot -> head through the
  // plan's work-balanced head order
  const int64_t per_xcd = gridDim.x / 8;
  const int64_t logical = static_cast<int64_t>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  const int64_t slot = logical / tiles_per_head;
  const int32_t tile = static_cast<int32_t>(logical - slot * tiles_per_head);
  if (!plan_matches(plan, bh_q / group, qn, kn, s_q)) {
    fill_nan_output(out, lse, bh_q, s_q, D, nan_pair<F16>());
    return;
  }
  if (slot >= bh_q) return;
  const int64_t bhkv = head_order_at(const_cast<int32_t*>(plan), bh_q / group, qn, kn)[slot / group];
  const int64_t bhq = bhkv * group + slot % group;
  PlanView pv = plan_at(const_cast<int32_t*>(plan), bhkv, qn, kn);
  // tiles of a head in decreasing q-cluster key count (the plan's tile2_sorted order)
  if (tile >= pv.tile2_sorted[qn]) return;
  int lo = 0, hi = qn;  // largest i with tile2_sorted[i] <= tile
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (pv.tile2_sorted[mid] <= tile) lo = mid; else hi = mid;
  }
  const int qc = pv.qc_by_len[lo];
  const int32_t row0 = pv.q_off[qc] + (tile - pv.tile2_sorted[lo]) * TBM;
  const int32_t row1 = min(row0 + TBM, pv.q_off[qc + 1]);
  // A tile with three or four live 32-row blocks pairs its waves: wave w (< 4) takes the
  // first 32-key half of every chunk for block w and wave w + 4 the second half, each with
  // its own online softmax, merged at the end (split-key helpers).  A tile with one or two
  // live blocks ("duo") walks its chunks two at a time: wave w takes block w & 1, half
  // (w >> 1) & 1 of chunk 2j + (w >> 2) in step j, so each block's keys are shared by four
  // waves, merged at the end.  Otherwise wave w owns block w and both halves.
  const int nblk = (row1 - row0 + 31) / 32;
  const bool duo = nblk <= 2;
  const bool split = !duo && nblk <= NW / 2;
  const int blk = duo ? (wave & 1) : split ? (wave & (NW / 2 - 1)) : wave;
  const int only = duo ? ((wave >> 1) & 1) : split ? (wave / (NW / 2)) : 0;  // the half a wave processes
  const int duo_part = wave >> 1;  // duo: 0 .. 3 = half + 2 (chunk parity); part 0 merges
  const bool wave_live = blk < nblk;
  const Seg* segs = pv.segs + static_cast<int64_t>(qc) * kn;
  const int32_t nseg = pv.nseg[qc];
  const int32_t total = pv.total[qc];

  const uint16_t* qb = q + bhq * static_cast<int64_t>(s_q) * D;
  const int32_t kv_bytes = s_kv * D * 2;
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(k + bhkv * static_cast<int64_t>(s_kv) * D), 0, kv_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(v + bhkv * static_cast<int64_t>(s_kv) * D), 0, kv_bytes, 0x00020000);
  if constexpr (SEGL) {
    for (int i = tid; i < nseg; i += NT) seg_lds[i] = segs[i];
  }

  int32_t my_row = row0 + blk * 32 + col;
  bool row_live = my_row < row1;
  if (q_index != nullptr && row_live) {
    my_row = q_index[bhq * static_cast<int64_t>(s_q) + my_row];
    row_live = my_row >= 0 && my_row < s_q;
  }
  u32x4 qf[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    qf[s] = row_live ? *reinterpret_cast<const u32x4*>(qb + static_cast<int64_t>(my_row) * D + s * 16 + half * 8)
                     : u32x4{0, 0, 0, 0};
  }
  spr::f32x16 o_acc[DBLK];
#pragma unroll
  for (int b = 0; b < DBLK; ++b) o_acc[b] = spr::f32x16{};
  float m_run = -__builtin_huge_valf();
  float l_run = 0.0f;
  // kept beside m_run and changed only when it moves: the exponent offset (0 while the
  // row has seen no finite score) and the lazy-rescale threshold
  float neg_m = 0.0f;
  float m_thr = -__builtin_huge_valf();

  const int nch = (total + BN - 1) / BN;

  int32_t cur_s = 0;
  auto plan_chunk = [&](int c) {
    if (wave == 0) {
      const int32_t vpos = min(c * BN + lane, total - 1);
      int32_t s = cur_s;
      if constexpr (SEGL) {
        while (s < nseg - 1 && vpos >= seg_lds[s].vend) ++s;
      } else {
        while (s < nseg - 1 && vpos >= segs[s].vend) ++s;
      }
      int32_t delta;
      if constexpr (SEGL) delta = seg_lds[s].delta; else delta = segs[s].delta;
      if constexpr (KIDX) {
        key_rows[c % 4][lane] = k_index[bhkv * static_cast<int64_t>(s_kv) + delta + vpos];
      } else {
        key_rows[c % 4][lane] = delta + vpos;
      }
      cur_s = __builtin_amdgcn_readlane(s, 63);
    }
  };
  int32_t krow[DMA_PER_WAVE];
  auto load_rows = [&](int c) {
    const int32_t* kr = key_rows[c % 4];
#pragma unroll
    for (int i = 0; i < DMA_PER_WAVE; ++i) krow[i] = kr[4 * wave + 4 * NW * i + (lane >> 4)];
  };
  auto dma = [&](uint8_t* kt, uint8_t* vt) {
    const int slot = lane & 15;
#pragma unroll
    for (int i = 0; i < DMA_PER_WAVE; ++i) {
      const int r0 = 4 * wave + 4 * NW * i;
      const int row = r0 + (lane >> 4);
      const int32_t off = krow[i] * DROW;
      lds_dma16(k_rsrc, kt + r0 * DROW, off + ((slot ^ (row & 15)) << 4));
      lds_dma16(v_rsrc, vt + r0 * DROW, off + ((slot ^ ((row & 3) << 2)) << 4));
    }
  };

  const int k_x = half ^ (col & 15);
  const int tr_a = lane & 3, tr_i = (lane >> 2) & 3, tr_g = (lane >> 4) & 1;
  const int v_lane = (4 * half + tr_i) * DROW + (tr_a & 1) * 8;
  const int v_piece = 2 * tr_g + (tr_a >> 1);
  const int v_x = 4 * tr_i;

  auto s_mma = [&](spr::f32x16& acc, const uint8_t* kt, int kbk) {
    acc = spr::f32x16{};
    const uint8_t* arow = kt + (kbk * 32 + col) * DROW;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(arow + (((2 * s) ^ k_x) << 4));
      acc = mfma16<F16>(a, qf[s], acc);
    }
  };
  // Row max of half kbk (masked past the end) and lazy rescale; returns -m.
  auto row_max = [&](spr::f32x16& acc, int kbk, int32_t left) {
    if (left < BN) {
      // element e holds key kbk * 32 + 8 (e / 4) + 4 half + e % 4; compared as an
      // immediate against one per-lane limit, so no per-element key registers
      const int lim = left - kbk * 32 - 4 * half;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        if (8 * (e / 4) + (e % 4) >= lim) acc[e] = -__builtin_huge_valf();
      }
    }
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, acc[e]);
    const float mloc = max_xor32_scaled(mx, scale_log2);
    const bool up = mloc > m_thr;
    if (__ballot(up) != 0ull) {
      // only the rows whose maximum grew move theirs: a row's result does not depend on
      // the other rows of its wave
      const float m_new = up ? mloc : m_run;
      const float alpha = up ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
      l_run *= alpha;
#pragma unroll
      for (int b = 0; b < DBLK; ++b) {
#pragma unroll
        for (int e = 0; e < 16; ++e) o_acc[b][e] *= alpha;
      }
      m_run = m_new;
      m_thr = m_new + RESCALE_SLACK;
      neg_m = (m_new == -__builtin_huge_valf()) ? 0.0f : -m_new;
    }
  };
  // One straight-line block: S^T of the next half into acc_next (K tile kt_n,
  // half kbk_n), interleaved step by step with P = 2^(s - m) of the current half
  // (acc) and its row sum, then O^T += V^T P^T over the current half's keys
  // (V tile vt, half kbk).  Fragments are read two steps ahead; the MFMAs of
  // S(h + 1) do not depend on the exponentials of half h, so the matrix unit and
  // the VALU work side by side.
  auto step = [&](spr::f32x16& acc_next, const uint8_t* kt_n, int kbk_n, const spr::f32x16& acc, const uint8_t* vt,
                  int kbk) {
    uint32_t pf[2][4];
    float lsum0 = 0.0f, lsum1 = 0.0f;
    acc_next = spr::f32x16{};
    const uint8_t* arow = kt_n + (kbk_n * 32 + col) * DROW;
    auto kfrag = [&](int st) { return *reinterpret_cast<const u32x4*>(arow + (((2 * st) ^ k_x) << 4)); };
    u32x4 ka[3];
    ka[0] = kfrag(0);
    ka[1] = kfrag(1);
#pragma unroll
    for (int st = 0; st < KSTEPS; ++st) {
      if (st + 2 < KSTEPS) ka[(st + 2) % 3] = kfrag(st + 2);
      acc_next = mfma16<F16>(ka[st % 3], qf[st], acc_next);
      const int e = 2 * st;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[e], scale_log2, neg_m));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[e + 1], scale_log2, neg_m));
      const uint32_t pk = pack2t<F16>(p0, p1);
      pf[e / 8][(e % 8) / 2] = pk;
      if (e % 4 == 0) {
        lsum0 = dot2_ones<F16>(pk, lsum0);
      } else {
        lsum1 = dot2_ones<F16>(pk, lsum1);
      }
    }
    l_run += lsum0 + lsum1;
    auto vfrag = [&](int f) {  // f = 4 tt + b
      const uint8_t* vrow = vt + 16 * (kbk * 2 + f / DBLK) * DROW + v_lane + (((4 * (f % DBLK) + v_piece) ^ v_x) << 4);
      const u32x2 r0 = lds_read_tr16(vrow);
      const u32x2 r1 = lds_read_tr16(vrow + 8 * DROW);
      return u32x4{r0.x, r0.y, r1.x, r1.y};
    };
    u32x4 va[3];
    va[0] = vfrag(0);
    va[1] = vfrag(1);
#pragma unroll
    for (int f = 0; f < 2 * DBLK; ++f) {
      if (f + 2 < 2 * DBLK) va[(f + 2) % 3] = vfrag(f + 2);
      const int tt = f / DBLK;
      const u32x4 bfrag = u32x4{pf[tt][0], pf[tt][1], pf[tt][2], pf[tt][3]};
      o_acc[f % DBLK] = mfma16<F16>(va[f % 3], bfrag, o_acc[f % DBLK]);
    }
  };

  // P = 2^(s - m) of half kbk (acc) and its row sum, then O^T += V^T P^T over that half's
  // keys: a step with no next S to overlap (duo tiles).
  auto pv_step = [&](const spr::f32x16& acc, const uint8_t* vt, int kbk) {
    uint32_t pf[2][4];
    float lsum0 = 0.0f, lsum1 = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[e], scale_log2, neg_m));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[e + 1], scale_log2, neg_m));
      const uint32_t pk = pack2t<F16>(p0, p1);
      pf[e / 8][(e % 8) / 2] = pk;
      if (e % 4 == 0) {
        lsum0 = dot2_ones<F16>(pk, lsum0);
      } else {
        lsum1 = dot2_ones<F16>(pk, lsum1);
      }
    }
    l_run += lsum0 + lsum1;
#pragma unroll
    for (int f = 0; f < 2 * DBLK; ++f) {
      const uint8_t* vrow = vt + 16 * (kbk * 2 + f / DBLK) * DROW + v_lane + (((4 * (f % DBLK) + v_piece) ^ v_x) << 4);
      const u32x2 r0 = lds_read_tr16(vrow);
      const u32x2 r1 = lds_read_tr16(vrow + 8 * DROW);
      const int tt = f / DBLK;
      const u32x4 bfrag = u32x4{pf[tt][0], pf[tt][1], pf[tt][2], pf[tt][3]};
      o_acc[f % DBLK] = mfma16<F16>(u32x4{r0.x, r0.y, r1.x, r1.y}, bfrag, o_acc[f % DBLK]);
    }
  };

  spr::f32x16 s_a, s_b;  // S^T of the current half / of the next half
  // Chunk x in tiles kt/vt; kt1 = K tile of chunk x + 1; kt3/vt3 (the tiles of
  // chunk x - 1) receive chunk x + 3.  The last chunk's second half still
  // computes a next S (from a stale buffer, unused) so that every block is the
  // same straight-line code.
  auto chunk = [&](int x, const uint8_t* kt, const uint8_t* vt, const uint8_t* kt1, uint8_t* kt3, uint8_t* vt3) {
    const int32_t left = total - x * BN;
    // ---- first half (S in s_a); S of the second half goes to s_b
    if (wave_live) {
      row_max(s_a, 0, left);
      step(s_b, kt, 1, s_a, vt, 0);
    }
    if (x + 4 < nch) plan_chunk(x + 4);
    if (x + 3 < nch) load_rows(x + 3);
    // ---- second half (S in s_b); S of the next chunk's first half goes to s_a
    if (wave_live) row_max(s_b, 1, left);
    // this wave's DMA of chunk x + 1 landed (that of chunk x + 2, issued later, may not have)
    if (x + 2 < nch) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DMA_PER_WAVE) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();  // ... every wave's; and no wave reads chunk x - 1 any more
    if (wave_live) step(s_a, kt1, 0, s_b, vt, 1);
    // chunk x + 3 into chunk x - 1's tiles, issued after this chunk's compute rather than
    // at the barrier, where every wave starts reading the next K tile (same-box timing:
    // about 2 % faster)
    if (x + 3 < nch) dma(kt3, vt3);
  };

  if (nch > 0 && duo) {
    // Step j computes chunks 2j and 2j + 1 (buffers (2j) & 3, (2j + 1) & 3) while chunks
    // 2j + 2 and 2j + 3 land in the other two buffers, whose chunks the step before
    // finished; key rows are planned four chunks ahead.
    if constexpr (SEGL) __syncthreads();  // staged segment list visible to wave 0
    for (int c = 0; c < 4 && c < nch; ++c) plan_chunk(c);
    __syncthreads();
    load_rows(0);
    dma(k_tile0, v_tile0);
    if (nch > 1) {
      load_rows(1);
      dma(k_tile1, v_tile1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    for (int x = 0; x < nch; x += 2) {
      __syncthreads();  // chunks x, x + 1 landed for every wave; chunks x - 2, x - 1 are done
      if (x + 2 < nch) {
        load_rows(x + 2);
        dma(k_tiles[(x + 2) & 3], v_tiles[(x + 2) & 3]);
      }
      if (x + 3 < nch) {
        load_rows(x + 3);
        dma(k_tiles[(x + 3) & 3], v_tiles[(x + 3) & 3]);
      }
      const int c = x + (duo_part >> 1);
      if (wave_live && c < nch) {
        s_mma(s_a, k_tiles[c & 3], only);
        row_max(s_a, only, total - c * BN);
        pv_step(s_a, v_tiles[c & 3], only);
      }
      if (x + 4 < nch) plan_chunk(x + 4);
      if (x + 5 < nch) plan_chunk(x + 5);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's chunks x + 2, x + 3 landed
    }
  } else if (nch > 0) {
    if constexpr (SEGL) __syncthreads();  // staged segment list visible to wave 0
    for (int c = 0; c < 4 && c < nch; ++c) plan_chunk(c);
    __syncthreads();
    load_rows(0);
    dma(k_tile0, v_tile0);
    if (nch > 1) {
      load_rows(1);
      dma(k_tile1, v_tile1);
    }
    if (nch > 2) {
      load_rows(2);
      dma(k_tile2, v_tile2);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // chunks 0 .. 2 landed
    if (wave_live) s_mma(s_a, k_tile0, only);
    if (split) {
      // One half per chunk: S of this wave's half of chunk x is in s_a; S of the same half
      // of chunk x + 1 (the next K tile, so after the barrier) goes to s_b.  The barriers,
      // DMAs and planning are those of the full path.
      for (int x = 0; x < nch; ++x) {
        const int32_t left = total - x * BN;
        if (x + 4 < nch) plan_chunk(x + 4);
        if (x + 3 < nch) load_rows(x + 3);
        if (wave_live) row_max(s_a, only, left);
        if (x + 2 < nch) {
          asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DMA_PER_WAVE) : "memory");
        } else {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
        if (wave_live) {
          step(s_b, k_tiles[(x + 1) & 3], only, s_a, v_tiles[x & 3], only);
          s_a = s_b;
        }
        if (x + 3 < nch) dma(k_tiles[(x + 3) & 3], v_tiles[(x + 3) & 3]);
      }
    } else {
      for (int x = 0; x < nch; x += 4) {
        chunk(x, k_tile0, v_tile0, k_tile1, k_tile3, v_tile3);
        if (x + 1 < nch) chunk(x + 1, k_tile1, v_tile1, k_tile2, k_tile0, v_tile0);
        if (x + 2 < nch) chunk(x + 2, k_tile2, v_tile2, k_tile3, k_tile1, v_tile1);
        if (x + 3 < nch) chunk(x + 3, k_tile3, v_tile3, k_tile0, k_tile2, v_tile2);
      }
    }
  }

  // ---- epilogue
  if (duo) {
    // parts 1 .. 3 of block b hand (m, l, O) to part 0 (wave b) through the K/V tiles:
    // O of (b, part) in slot 3 b + part - 1 (16 KB each: k_tiles[0..3], v_tiles[0..1]),
    // m and l in v_tiles[3]; part 0 adds them in part order
    __syncthreads();  // every wave is past its last chunk
    auto o_slot = [&](int b, int pt) {
      const int sl = 3 * b + pt - 1;
      return reinterpret_cast<float*>(sl < 4 ? k_tiles[sl] : v_tiles[sl - 4]);
    };
    float* ml = reinterpret_cast<float*>(v_tiles[3]);
    if (duo_part != 0 && wave_live) {
      float* po = o_slot(blk, duo_part) + lane * (DBLK * 16);
#pragma unroll
      for (int b = 0; b < DBLK; ++b) {
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
          *reinterpret_cast<spr::f32x4*>(po + b * 16 + e) =
              spr::f32x4{o_acc[b][e], o_acc[b][e + 1], o_acc[b][e + 2], o_acc[b][e + 3]};
        }
      }
      ml[((3 * blk + duo_part - 1) * 64 + lane) * 2] = m_run;
      ml[((3 * blk + duo_part - 1) * 64 + lane) * 2 + 1] = l_run;
    }
    __syncthreads();
    if (duo_part != 0) {
      row_live = false;  // part 0 writes the block
    } else if (wave_live) {
      float mm = m_run;
#pragma unroll
      for (int pt = 1; pt < 4; ++pt) mm = fmaxf(mm, ml[((3 * blk + pt - 1) * 64 + lane) * 2]);
      const float a0 = m_run == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(m_run - mm);
      l_run *= a0;
#pragma unroll
      for (int b = 0; b < DBLK; ++b) {
#pragma unroll
        for (int e = 0; e < 16; ++e) o_acc[b][e] *= a0;
      }
#pragma unroll
      for (int pt = 1; pt < 4; ++pt) {
        const float mi = ml[((3 * blk + pt - 1) * 64 + lane) * 2];
        const float li = ml[((3 * blk + pt - 1) * 64 + lane) * 2 + 1];
        const float ai = mi == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(mi - mm);
        const float* po = o_slot(blk, pt) + lane * (DBLK * 16);
#pragma unroll
        for (int b = 0; b < DBLK; ++b) {
#pragma unroll
          for (int e = 0; e < 16; e += 4) {
            const spr::f32x4 oi = *reinterpret_cast<const spr::f32x4*>(po + b * 16 + e);
#pragma unroll
            for (int j = 0; j < 4; ++j) o_acc[b][e + j] += oi[j] * ai;
          }
        }
        l_run += li * ai;
      }
      m_run = mm;
    }
  }
  if (split) {
    // wave w + 4 hands its (m, l, O) for the second halves to wave w through the K/V tiles
    // (every wave is past its last chunk after the barrier)
    __syncthreads();
    uint8_t* const kt_m = k_tiles[blk];
    float* ml = reinterpret_cast<float*>(v_tile0);
    if (only == 1 && wave_live) {
      float* po = reinterpret_cast<float*>(kt_m) + lane * (DBLK * 16);
#pragma unroll
      for (int b = 0; b < DBLK; ++b) {
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
          *reinterpret_cast<spr::f32x4*>(po + b * 16 + e) =
              spr::f32x4{o_acc[b][e], o_acc[b][e + 1], o_acc[b][e + 2], o_acc[b][e + 3]};
        }
      }
      ml[(blk * 64 + lane) * 2] = m_run;
      ml[(blk * 64 + lane) * 2 + 1] = l_run;
    }
    __syncthreads();
    if (only == 1) {
      row_live = false;  // the first-half wave writes the block
    } else if (wave_live) {
      const float* po = reinterpret_cast<const float*>(kt_m) + lane * (DBLK * 16);
      const float m1 = ml[(blk * 64 + lane) * 2], l1 = ml[(blk * 64 + lane) * 2 + 1];
      const float mm = fmaxf(m_run, m1);
      const float a0 = m_run == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(m_run - mm);
      const float a1 = m1 == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
#pragma unroll
      for (int b = 0; b < DBLK; ++b) {
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
          const spr::f32x4 o1 = *reinterpret_cast<const spr::f32x4*>(po + b * 16 + e);
#pragma unroll
          for (int j = 0; j < 4; ++j) o_acc[b][e + j] = o_acc[b][e + j] * a0 + o1[j] * a1;
        }
      }
      l_run = l_run * a0 + l1 * a1;
      m_run = mm;
    }
  }
  const float l_tot = sum_xor32(l_run);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (row_live) {
    uint16_t* orow = out + (bhq * static_cast<int64_t>(s_q) + my_row) * D;
#pragma unroll
    for (int b = 0; b < DBLK; ++b) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d0 = b * 32 + 8 * i + 4 * half;
        uint2 w;
        w.x = pack2t<F16>(o_acc[b][4 * i] * inv, o_acc[b][4 * i + 1] * inv);
        w.y = pack2t<F16>(o_acc[b][4 * i + 2] * inv, o_acc[b][4 * i + 3] * inv);
        *reinterpret_cast<uint2*>(orow + d0) = w;
      }
    }
    if (lse != nullptr && half == 0) {
      lse[bhq * static_cast<int64_t>(s_q) + my_row] =
          l_tot > 0.0f ? (m_run + __builtin_amdgcn_logf(l_tot)) * 0.69314718055994531f : -__builtin_huge_valf();
    }
  }
}

// Merge split-key partials: out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s.
// One thread per (bhq, row, 4 dims).  out_dtype 0 = bf16, 1 = fp16, 2 = fp32.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ part_o,
                                                           const float* __restrict__ part_ml, int64_t rows_total,
                                                           int32_t s_q, int32_t nsplit, int32_t out_dtype,
                                                           void* __restrict__ out, float* __restrict__ lse) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t r = g / (D / 4);
  const int d0 = static_cast<int>(g % (D / 4)) * 4;
  if (r >= rows_total) return;
  const int64_t bhq = r / s_q;
  const int64_t row = r - bhq * s_q;
  float mx = -__builtin_huge_valf();
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, part_ml[((bhq * nsplit + s) * s_q + row) * 2]);
  const float mu = (mx == -__builtin_huge_valf()) ? 0.0f : mx;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float l = 0.0f;
  for (int s = 0; s < nsplit; ++s) {
    const int64_t slot = (bhq * nsplit + s) * s_q + row;
    const float w = __builtin_amdgcn_exp2f(part_ml[slot * 2] - mu);
    l += w * part_ml[slot * 2 + 1];
    const spr::f32x4 o = *reinterpret_cast<const spr::f32x4*>(part_o + slot * D + d0);
    acc[0] += w * o[0];
    acc[1] += w * o[1];
    acc[2] += w * o[2];
    acc[3] += w * o[3];
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  if (out_dtype == 0 || out_dtype == 1) {
    uint2 w;
    w.x = out_dtype == 0 ? pack2(acc[0] * inv, acc[1] * inv) : pack2t<true>(acc[0] * inv, acc[1] * inv);
    w.y = out_dtype == 0 ? pack2(acc[2] * inv, acc[3] * inv) : pack2t<true>(acc[2] * inv, acc[3] * inv);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + r * D + d0) = w;
  } else {
    *reinterpret_cast<spr::f32x4*>(static_cast<float*>(out) + r * D + d0) =
        spr::f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
  }
  if (lse != nullptr && d0 == 0) {
    lse[r] = l > 0.0f ? (mu + __builtin_amdgcn_logf(l)) * 0.69314718055994531f : -__builtin_huge_valf();
  }
}

}  // namespace

// ------------------------------------------------------------------------------ C ABI

// Order of the kv heads over the tile grid of attn_pipe_kernel.  The hardware hands
// workgroup i to XCD i % 8 and the kernel gives each XCD a contiguous run of heads
// (bh_kv / 8 kv heads), so an XCD whose heads keep more key pairs finishes last.  The
// work of a head is sum over q-clusters of 256-row tiles x 64-key chunks; in descending
// order of work (ties by index) each head goes to the XCD with the least work so far
// among those with a free slot (longest-processing-time first, bh_kv / 8 heads each).
// Identity when bh_kv is not a multiple of 8 or above HO_MAX heads.  One workgroup.
constexpr int HO_MAX = 1024;
constexpr int TO_MAX_QN = 4096;  // q-clusters per head the tile order handles in LDS

// Inside each head, the q-clusters by decreasing key count (ties by index), so that every
// XCD ends on its shortest tiles, and the first tile of each in that order.  One
// workgroup per kv head; key counts, tile counts and the order staged in LDS.
__global__ __launch_bounds__(256) void attn_tile_order_kernel(int32_t* __restrict__ plan, int32_t qn, int32_t kn) {
  extern __shared__ int32_t to_lds[];  // total[qn], tiles[qn], by_len[qn]
  int32_t* tl = to_lds;
  int32_t* tc = to_lds + qn;
  int32_t* by_len = to_lds + 2 * qn;
  const PlanView pv = plan_at(plan, blockIdx.x, qn, kn);
  const int tid = threadIdx.x;
  for (int qc = tid; qc < qn; qc += blockDim.x) {
    tl[qc] = pv.total[qc];
    tc[qc] = pv.tile2_off[qc + 1] - pv.tile2_off[qc];
  }
  __syncthreads();
  for (int qc = tid; qc < qn; qc += blockDim.x) {
    const int32_t t = tl[qc];
    int rank = 0;
    for (int o = 0; o < qn; ++o) rank += (tl[o] > t || (tl[o] == t && o < qc)) ? 1 : 0;
    by_len[rank] = qc;
    pv.qc_by_len[rank] = qc;
  }
  __syncthreads();
  if (tid == 0) {
    int32_t run = 0;
    for (int r = 0; r < qn; ++r) {
      pv.tile2_sorted[r] = run;
      run += tc[by_len[r]];
    }
    pv.tile2_sorted[qn] = run;
  }
}
__global__ __launch_bounds__(256) void attn_head_order_kernel(int32_t* __restrict__ plan, int32_t bh_kv, int32_t qn,
                                                              int32_t kn) {
  __shared__ int64_t work[HO_MAX];
  __shared__ int16_t by_rank[HO_MAX];
  int32_t* order = head_order_at(plan, bh_kv, qn, kn);
  const int tid = threadIdx.x;
  if (bh_kv % 8 != 0 || bh_kv > HO_MAX) {
    for (int h = tid; h < bh_kv; h += blockDim.x) order[h] = h;
    return;
  }
  for (int h = tid; h < bh_kv; h += blockDim.x) work[h] = 0;
  __syncthreads();
  // (head, q-cluster) terms spread over the workgroup, summed with LDS atomics (integers:
  // the order does not matter)
  for (int64_t i = tid; i < static_cast<int64_t>(bh_kv) * qn; i += blockDim.x) {
    const int h = static_cast<int>(i / qn), qc = static_cast<int>(i % qn);
    const PlanView pv = plan_at(plan, h, qn, kn);
    const int64_t w = static_cast<int64_t>(pv.tile2_off[qc + 1] - pv.tile2_off[qc]) * ((pv.total[qc] + BN - 1) / BN);
    if (w != 0) atomicAdd(reinterpret_cast<unsigned long long*>(&work[h]), static_cast<unsigned long long>(w));
  }
  __syncthreads();
  for (int h = tid; h < bh_kv; h += blockDim.x) {
    int rank = 0;
    for (int o = 0; o < bh_kv; ++o) rank += (work[o] > work[h] || (work[o] == work[h] && o < h)) ? 1 : 0;
    by_rank[rank] = static_cast<int16_t>(h);
  }
  __syncthreads();
  if (tid == 0) {
    const int hpx = bh_kv / 8;
    int64_t load[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int used[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int rank = 0; rank < bh_kv; ++rank) {
      const int h = by_rank[rank];
      int best = -1;
      for (int x = 0; x < 8; ++x) {
        if (used[x] < hpx && (best < 0 || load[x] < load[best])) best = x;
      }
      order[best * hpx + used[best]] = h;
      ++used[best];
      load[best] += work[h];
    }
  }
}

// Written after the rest of the plan (stream order), so a run that sees a matching
// header sees the finished plan.
__global__ void attn_plan_header_kernel(int32_t* __restrict__ plan, int32_t bh_kv, int32_t qn, int32_t kn,
                                        int32_t s) {
  int32_t* hd = head_order_at(plan, bh_kv, qn, kn) + bh_kv;
  if (threadIdx.x == 0) {
    hd[0] = PLAN_MAGIC;
    hd[1] = bh_kv;
    hd[2] = qn;
    hd[3] = kn;
    hd[4] = s;
  }
}

extern "C" size_t spr_block_sparse_attention_workspace(int64_t bh_kv, int32_t qn, int32_t kn) {
  return static_cast<size_t>((bh_kv * plan_words(qn, kn) + bh_kv + PLAN_HEADER_WORDS) * 4);
}

// Plan for spr_block_sparse_attention_run: map uint8 [bh_kv, qn, kn], q_sizes
// [bh_kv, qn], k_sizes [bh_kv, kn] int32 (sizes are clamped to the s rows).
static int block_sparse_plan(const uint8_t* map, const int32_t* ids, const int32_t* counts, const int32_t* q_sizes,
                             const int32_t* k_sizes, int64_t bh_kv, int64_t s, int32_t qn, int32_t kn, void* plan,
                             size_t plan_bytes, hipStream_t stream) {
  SPR_REQUIRE(bh_kv >= 1 && s >= 0 && qn >= 1 && kn >= 1, "spr_block_sparse_attention_plan: bad size");
  SPR_REQUIRE(kn <= 16384, "spr_block_sparse_attention_plan: kn exceeds 16384");
  SPR_REQUIRE(qn <= TO_MAX_QN, "spr_block_sparse_attention_plan: qn exceeds %d", TO_MAX_QN);
  SPR_REQUIRE(s < (int64_t(1) << 31), "spr_block_sparse_attention_plan: sequence too long");
  SPR_REQUIRE(bh_kv <= 65535, "spr_block_sparse_attention_plan: bh_kv exceeds 65535");
  SPR_REQUIRE((map != nullptr) != (ids != nullptr && counts != nullptr),
              "spr_block_sparse_attention_plan: give a map or a schedule (ids and counts)");
  SPR_REQUIRE(q_sizes && k_sizes && plan, "spr_block_sparse_attention_plan: null pointer");
  const size_t need = spr_block_sparse_attention_workspace(bh_kv, qn, kn);
  if (plan_bytes < need) {
    spr_set_error("spr_block_sparse_attention_plan: plan buffer %zu < %zu bytes", plan_bytes, need);
    return SPR_EWORKSPACE;
  }
  // one wave per q-cluster row: the rows of a head spread over several workgroups
  const uint32_t row_groups = static_cast<uint32_t>(spr::ceil_div(qn, THREADS / 64));
  const size_t koff_bytes = (kn + 1) * sizeof(int32_t);  // up to 65540 bytes at kn = 16384
  if (koff_bytes > 65536) {
    static bool raised = false;  // the attribute is per kernel, per process
    if (!raised) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_plan_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 16384 * 4 + 4);
      if (e != hipSuccess) {
        spr_set_error("spr_block_sparse_attention_plan: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
        return SPR_ELAUNCH;
      }
      raised = true;
    }
  }
  attn_plan_kernel<<<dim3(static_cast<uint32_t>(bh_kv), row_groups), THREADS, koff_bytes, stream>>>(
      map, ids, counts, q_sizes, k_sizes, qn, kn, static_cast<int32_t>(s), static_cast<int32_t*>(plan));
  SPR_LAUNCHED("attn_plan_kernel");
  attn_tile_order_kernel<<<dim3(static_cast<uint32_t>(bh_kv)), 256, 3 * qn * sizeof(int32_t), stream>>>(
      static_cast<int32_t*>(plan), qn, kn);
  SPR_LAUNCHED("attn_tile_order_kernel");
  attn_head_order_kernel<<<1, 256, 0, stream>>>(static_cast<int32_t*>(plan), static_cast<int32_t>(bh_kv), qn, kn);
  SPR_LAUNCHED("attn_head_order_kernel");
  attn_plan_header_kernel<<<1, 64, 0, stream>>>(static_cast<int32_t*>(plan), static_cast<int32_t>(bh_kv), qn, kn,
                                                static_cast<int32_t>(s));
  SPR_LAUNCHED("attn_plan_header_kernel");
  return SPR_OK;
}

extern "C" int spr_block_sparse_attention_plan(const uint8_t* map, const int32_t* q_sizes, const int32_t* k_sizes,
                                               int64_t bh_kv, int64_t s, int32_t qn, int32_t kn, void* plan,
                                               size_t plan_bytes, hipStream_t stream) {
  SPR_REQUIRE(map != nullptr, "spr_block_sparse_attention_plan: null map");
  return block_sparse_plan(map, nullptr, nullptr, q_sizes, k_sizes, bh_kv, s, qn, kn, plan, plan_bytes, stream);
}

// The plan from a selector schedule: ids int32 [bh_kv, qn, kn] (row r's first counts[r]
// entries are its kept k-clusters, strictly ascending), counts int32 [bh_kv, qn].
extern "C" int spr_block_sparse_attention_plan_schedule(const int32_t* ids, const int32_t* counts,
                                                        const int32_t* q_sizes, const int32_t* k_sizes,
                                                        int64_t bh_kv, int64_t s, int32_t qn, int32_t kn, void* plan,
                                                        size_t plan_bytes, hipStream_t stream) {
  SPR_REQUIRE(ids != nullptr && counts != nullptr, "spr_block_sparse_attention_plan_schedule: null schedule");
  return block_sparse_plan(nullptr, ids, counts, q_sizes, k_sizes, bh_kv, s, qn, kn, plan, plan_bytes, stream);
}

// q [bh_q, s, d], k/v [bh_kv, s, d] (cluster-contiguous) of dtype 0 bf16 / 1 fp16, plan from
// spr_block_sparse_attention_plan; out [bh_q, s, d] of the same dtype; lse fp32 [bh_q, s]
// (nullable, natural log).  d in {16, 32, 64, 128}.  bh_q must be a multiple of bh_kv (GQA
// groups).  q_index int32 [bh_q, s] (nullable): q, out and lse stay in token order and
// cluster-sorted row r is token q_index[r] (the Q permutation and its inverse fused into the
// attention).  k_index int32 [bh_kv, s] (nullable): k and v stay in token order and
// cluster-sorted key position p is token k_index[p] (the K/V permutation fused into the key
// gather).
extern "C" int spr_block_sparse_attention_run_ex(const void* q, const void* k, const void* v, const void* plan,
                                                 size_t plan_bytes, int64_t bh_q, int64_t bh_kv, int64_t s, int32_t d,
                                                 int32_t qn, int32_t kn, float scale, int32_t dtype,
                                                 const int32_t* q_index, const int32_t* k_index, void* out, float* lse,
                                                 hipStream_t stream) {
  SPR_REQUIRE(bh_q >= 0 && bh_kv >= 1 && s >= 0 && qn >= 1 && kn >= 1, "spr_block_sparse_attention_run: bad size");
  SPR_REQUIRE(bh_q % bh_kv == 0, "spr_block_sparse_attention_run: bh_q=%lld not a multiple of bh_kv=%lld",
              (long long)bh_q, (long long)bh_kv);
  SPR_REQUIRE(d == 16 || d == 32 || d == 64 || d == 128,
              "spr_block_sparse_attention_run: head dim %d not supported (16, 32, 64, 128)", d);
  SPR_REQUIRE(dtype == 0 || dtype == 1, "spr_block_sparse_attention_run: dtype must be 0 (bf16) or 1 (fp16), got %d",
              dtype);
  // the row maximum is taken on unscaled scores and then scaled, which needs scale > 0
  SPR_REQUIRE(scale > 0.0f && scale < __builtin_huge_valf(),
              "spr_block_sparse_attention_run: scale must be positive and finite (got %g)", double(scale));
  SPR_REQUIRE(s * d * 2 < (int64_t(1) << 31), "spr_block_sparse_attention_run: a head of K/V exceeds 2 GiB");
  SPR_REQUIRE(bh_q <= 65535, "spr_block_sparse_attention_run: bh_q exceeds 65535");
  if (bh_q == 0 || s == 0) return SPR_OK;
  SPR_REQUIRE(q && k && v && plan && out, "spr_block_sparse_attention_run: null pointer");
  SPR_REQUIRE(kn <= 16384 && qn <= TO_MAX_QN && bh_kv <= 65535, "spr_block_sparse_attention_run: bad plan size");
  {
    const size_t need = spr_block_sparse_attention_workspace(bh_kv, qn, kn);
    if (plan_bytes < need) {
      spr_set_error("spr_block_sparse_attention_run: plan buffer %zu < %zu bytes for bh_kv=%lld qn=%d kn=%d",
                    plan_bytes, need, (long long)bh_kv, qn, kn);
      return SPR_EWORKSPACE;
    }
  }
  SPR_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(v) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
              "spr_block_sparse_attention_run: q/k/v/out must be 16-byte aligned");
  const int64_t max_tiles = spr::ceil_div(s, BM) + qn;
  const int64_t blocks = spr::ceil_div(max_tiles * bh_q, 8) * 8;
  SPR_REQUIRE(blocks < (int64_t(1) << 31), "spr_block_sparse_attention_run: too many tiles");
  dim3 grid(static_cast<uint32_t>(blocks));
  const int32_t group = static_cast<int32_t>(bh_q / bh_kv);
  const float scale_log2 = scale * 1.4426950408889634f;
  const bool seg_lds = kn <= MAX_LDS_SEGS;
  const bool kx = k_index != nullptr;
  const bool f16 = dtype == 1;
  const uint16_t* q16 = static_cast<const uint16_t*>(q);
  const uint16_t* k16 = static_cast<const uint16_t*>(k);
  const uint16_t* v16 = static_cast<const uint16_t*>(v);
  const int32_t* pl = static_cast<const int32_t*>(plan);
  uint16_t* o16 = static_cast<uint16_t*>(out);
  const int32_t s32 = static_cast<int32_t>(s), bhq32 = static_cast<int32_t>(bh_q);
  if (d == 128) {
    const int64_t max_tiles_pipe = spr::ceil_div(s, 2 * BM) + qn;
    dim3 grid_pipe(static_cast<uint32_t>(spr::ceil_div(max_tiles_pipe * bh_q, 8) * 8));
    const int32_t tph = static_cast<int32_t>(max_tiles_pipe);
    auto pipe = [&](auto sl, auto kxc, auto f) {
      attn_pipe_kernel<decltype(sl)::value, decltype(kxc)::value, decltype(f)::value><<<grid_pipe, 512, 0, stream>>>(
          q16, k16, v16, s32, s32, group, qn, kn, pl, bhq32, tph, scale_log2, q_index, k_index, o16, lse);
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    if (seg_lds) {
      if (kx) { f16 ? pipe(T_{}, T_{}, T_{}) : pipe(T_{}, T_{}, F_{}); }
      else    { f16 ? pipe(T_{}, F_{}, T_{}) : pipe(T_{}, F_{}, F_{}); }
    } else {
      if (kx) { f16 ? pipe(F_{}, T_{}, T_{}) : pipe(F_{}, T_{}, F_{}); }
      else    { f16 ? pipe(F_{}, F_{}, T_{}) : pipe(F_{}, F_{}, F_{}); }
    }
    SPR_LAUNCHED("attn_pipe_kernel");
    return SPR_OK;
  }
  auto fwd = [&](auto dd, auto sl, auto kxc, auto f) {
    attn_fwd_kernel<decltype(dd)::value, 0, decltype(sl)::value, ATTN_NW, ATTN_QB, decltype(kxc)::value,
                    decltype(f)::value><<<grid, ATTN_NW * 64, 0, stream>>>(
        q16, k16, v16, s32, s32, group, qn, kn, pl, bhq32, static_cast<int32_t>(max_tiles), scale_log2, q_index,
        k_index, o16, lse, 0, nullptr, nullptr, s * decltype(dd)::value);
  };
  auto by_flags = [&](auto dd) {
    using T_ = std::true_type;
    using F_ = std::false_type;
    if (seg_lds) {
      if (kx) { f16 ? fwd(dd, T_{}, T_{}, T_{}) : fwd(dd, T_{}, T_{}, F_{}); }
      else    { f16 ? fwd(dd, T_{}, F_{}, T_{}) : fwd(dd, T_{}, F_{}, F_{}); }
    } else {
      if (kx) { f16 ? fwd(dd, F_{}, T_{}, T_{}) : fwd(dd, F_{}, T_{}, F_{}); }
      else    { f16 ? fwd(dd, F_{}, F_{}, T_{}) : fwd(dd, F_{}, F_{}, F_{}); }
    }
  };
  if (d == 64) by_flags(std::integral_constant<int, 64>{});
  else if (d == 32) by_flags(std::integral_constant<int, 32>{});
  else by_flags(std::integral_constant<int, 16>{});
  SPR_LAUNCHED("attn_fwd_kernel");
  return SPR_OK;
}

extern "C" int spr_block_sparse_attention_run(const void* q, const void* k, const void* v, const void* plan,
                                              size_t plan_bytes, int64_t bh_q, int64_t bh_kv, int64_t s, int32_t d,
                                              int32_t qn, int32_t kn, float scale, const int32_t* q_index,
                                              const int32_t* k_index, void* out, float* lse, hipStream_t stream) {
  return spr_block_sparse_attention_run_ex(q, k, v, plan, plan_bytes, bh_q, bh_kv, s, d, qn, kn, scale, 0, q_index,
                                           k_index, out, lse, stream);
}

// Plan + run in one call (workspace = plan buffer); dtype as spr_block_sparse_attention_run_ex.
extern "C" int spr_block_sparse_attention_ex(const void* q, const void* k, const void* v, const uint8_t* map,
                                             const int32_t* q_sizes, const int32_t* k_sizes, int64_t bh_q,
                                             int64_t bh_kv, int64_t s, int32_t d, int32_t qn, int32_t kn, float scale,
                                             int32_t dtype, const int32_t* q_index, const int32_t* k_index, void* out,
                                             float* lse, void* workspace, size_t workspace_bytes,
                                             hipStream_t stream) {
  if (bh_q == 0 || s == 0) return SPR_OK;
  int st = spr_block_sparse_attention_plan(map, q_sizes, k_sizes, bh_kv, s, qn, kn, workspace, workspace_bytes,
                                           stream);
  if (st != SPR_OK) return st;
  return spr_block_sparse_attention_run_ex(q, k, v, workspace, workspace_bytes, bh_q, bh_kv, s, d, qn, kn, scale,
                                           dtype, q_index, k_index, out, lse, stream);
}

// Plan + run in one call (workspace = plan buffer), bf16.
extern "C" int spr_block_sparse_attention(const void* q, const void* k, const void* v, const uint8_t* map,
                                          const int32_t* q_sizes, const int32_t* k_sizes, int64_t bh_q,
                                          int64_t bh_kv, int64_t s, int32_t d, int32_t qn, int32_t kn, float scale,
                                          const int32_t* q_index, const int32_t* k_index, void* out, float* lse,
                                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return spr_block_sparse_attention_ex(q, k, v, map, q_sizes, k_sizes, bh_q, bh_kv, s, d, qn, kn, scale, 0, q_index,
                                       k_index, out, lse, workspace, workspace_bytes, stream);
}

extern "C" size_t spr_dense_attention_workspace(int64_t bh_q, int64_t m, int32_t d, int32_t nsplit) {
  return static_cast<size_t>(bh_q * nsplit * m * (static_cast<int64_t>(d) + 2) * 4);
}

// Dense softmax(q k^T * scale) v for a few query rows per head (probe rows):
// q [bh_q, m, d] bf16, k/v [bh_kv, s_kv, d] bf16, keys split into nsplit ranges
// processed in parallel and merged.  out [bh_q, m, d] (out_dtype 0 = bf16, 2 = fp32),
// lse fp32 [bh_q, m] nullable.
extern "C" int spr_dense_attention_strided(const void* q, const void* k, const void* v, int64_t bh_q, int64_t bh_kv,
                                           int64_t m, int64_t s_kv, int64_t kv_head_stride, int32_t d, float scale,
                                           int32_t nsplit, void* out, int32_t out_dtype, float* lse, void* workspace,
                                           size_t workspace_bytes, hipStream_t stream);

extern "C" int spr_dense_attention(const void* q, const void* k, const void* v, int64_t bh_q, int64_t bh_kv,
                                   int64_t m, int64_t s_kv, int32_t d, float scale, int32_t nsplit, void* out,
                                   int32_t out_dtype, float* lse, void* workspace, size_t workspace_bytes,
                                   hipStream_t stream) {
  return spr_dense_attention_strided(q, k, v, bh_q, bh_kv, m, s_kv, s_kv * d, d, scale, nsplit, out, out_dtype, lse,
                                     workspace, workspace_bytes, stream);
}

// The same with kv head h's rows starting kv_head_stride elements after head h - 1's
// (rows of d contiguous elements, s_kv of them per head): a slice of the keys of a larger
// packed tensor is read in place.  q, k, v of dtype 0 bf16 / 1 fp16; d in {16, 32, 64, 128};
// out_dtype 0 bf16, 1 fp16, 2 fp32.
extern "C" int spr_dense_attention_strided_ex(const void* q, const void* k, const void* v, int64_t bh_q,
                                              int64_t bh_kv, int64_t m, int64_t s_kv, int64_t kv_head_stride,
                                              int32_t d, float scale, int32_t dtype, int32_t nsplit, void* out,
                                              int32_t out_dtype, float* lse, void* workspace, size_t workspace_bytes,
                                              hipStream_t stream) {
  SPR_REQUIRE(bh_q >= 0 && bh_kv >= 1 && m >= 0 && s_kv >= 0 && nsplit >= 1, "spr_dense_attention: bad size");
  SPR_REQUIRE(kv_head_stride >= s_kv * d, "spr_dense_attention: kv head stride %lld below s_kv * d",
              static_cast<long long>(kv_head_stride));
  SPR_REQUIRE(bh_q % bh_kv == 0, "spr_dense_attention: bh_q not a multiple of bh_kv");
  SPR_REQUIRE(d == 16 || d == 32 || d == 64 || d == 128, "spr_dense_attention: head dim %d not supported "
              "(16, 32, 64, 128)", d);
  SPR_REQUIRE(dtype == 0 || dtype == 1, "spr_dense_attention: dtype must be 0 (bf16) or 1 (fp16)");
  SPR_REQUIRE(out_dtype >= 0 && out_dtype <= 2, "spr_dense_attention: out_dtype must be 0, 1 or 2");
  SPR_REQUIRE(scale > 0.0f && scale < __builtin_huge_valf(),
              "spr_dense_attention: scale must be positive and finite (got %g)", double(scale));
  SPR_REQUIRE(s_kv * d * 2 < (int64_t(1) << 31) && m < (int64_t(1) << 31), "spr_dense_attention: too long");
  SPR_REQUIRE(bh_q <= 65535 && nsplit <= 65535, "spr_dense_attention: grid too large");
  if (bh_q == 0 || m == 0) return SPR_OK;
  SPR_REQUIRE(q && k && v && out && workspace, "spr_dense_attention: null pointer");
  const size_t need = spr_dense_attention_workspace(bh_q, m, d, nsplit);
  if (workspace_bytes < need) {
    spr_set_error("spr_dense_attention: workspace %zu < %zu bytes", workspace_bytes, need);
    return SPR_EWORKSPACE;
  }
  const int32_t split_len = static_cast<int32_t>(spr::ceil_div(s_kv, nsplit));
  float* part_o = static_cast<float*>(workspace);
  float* part_ml = part_o + bh_q * nsplit * m * d;
  dim3 grid(static_cast<uint32_t>(nsplit), static_cast<uint32_t>(spr::ceil_div(m, BM)),
            static_cast<uint32_t>(bh_q));
  const int32_t group = static_cast<int32_t>(bh_q / bh_kv);
  const float scale_log2 = scale * 1.4426950408889634f;
  const int64_t rows_total = bh_q * m;
  const uint32_t cblocks = static_cast<uint32_t>(spr::ceil_div(rows_total * (d / 4), 256));
  auto run = [&](auto dd, auto f) -> int {
    constexpr int DD = decltype(dd)::value;
    attn_fwd_kernel<DD, 1, false, 4, 1, false, decltype(f)::value><<<grid, THREADS, 0, stream>>>(
        static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
        static_cast<int32_t>(m), static_cast<int32_t>(s_kv), group, 0, 0, nullptr, static_cast<int32_t>(bh_q), 0,
        scale_log2, nullptr, nullptr, nullptr, nullptr, split_len, part_o, part_ml, kv_head_stride);
    SPR_LAUNCHED("attn_fwd_kernel(dense)");
    attn_combine_kernel<DD><<<cblocks, 256, 0, stream>>>(part_o, part_ml, rows_total, static_cast<int32_t>(m), nsplit,
                                                         out_dtype, out, lse);
    SPR_LAUNCHED("attn_combine_kernel");
    return SPR_OK;
  };
  auto by_dim = [&](auto f) -> int {
    if (d == 128) return run(std::integral_constant<int, 128>{}, f);
    if (d == 64) return run(std::integral_constant<int, 64>{}, f);
    if (d == 32) return run(std::integral_constant<int, 32>{}, f);
    return run(std::integral_constant<int, 16>{}, f);
  };
  return dtype == 1 ? by_dim(std::true_type{}) : by_dim(std::false_type{});
}

extern "C" int spr_dense_attention_strided(const void* q, const void* k, const void* v, int64_t bh_q, int64_t bh_kv,
                                           int64_t m, int64_t s_kv, int64_t kv_head_stride, int32_t d, float scale,
                                           int32_t nsplit, void* out, int32_t out_dtype, float* lse, void* workspace,
                                           size_t workspace_bytes, hipStream_t stream) {
  return spr_dense_attention_strided_ex(q, k, v, bh_q, bh_kv, m, s_kv, kv_head_stride, d, scale, 0, nsplit, out,
                                        out_dtype, lse, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------- allocation-free variant
// spr_block_sparse_attention with its plan in a fixed device array instead of a caller
// workspace, for callers that cannot allocate device memory (code under HIP graph
// capture, serving loops that forbid hipMalloc).  `scratch` holds one plan of at most
// NOALLOC_PLAN_BYTES: every BASELINE shape fits (C3 15.4 MiB, C4 12.1 MiB, C5 20.1 MiB,
// the N8 defaults of 300 x 1000 clusters at 24 heads 55.1 MiB).  Each device the library
// runs on holds its own copy until the process ends.  The host never names the array in
// a launch or copy: its device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and kept in g_scratch_addr.
// The plan kernels write every word the run reads (the header last), so nothing has to
// start at zero; calls that overlap on one device (two streams, two threads) share the
// array and race.
constexpr size_t NOALLOC_PLAN_BYTES = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_PLAN_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[NOALLOC_MAX_DEVICES] = {};

// Device address of this device's `scratch` (looked up on the first call per device).
int noalloc_scratch_addr(void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    spr_set_error("spr_block_sparse_attention_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return SPR_ELAUNCH;
  }
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
    spr_set_error("spr_block_sparse_attention_noalloc: device %d outside [0, %d)", dev, NOALLOC_MAX_DEVICES);
    return SPR_EINVAL;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      spr_set_error("spr_block_sparse_attention_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                    dev, hipGetErrorString(e));
      return SPR_ELAUNCH;
    }
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return SPR_OK;
}
}  // namespace

extern "C" int spr_block_sparse_attention_noalloc(const void* q, const void* k, const void* v, const uint8_t* map,
                                                  const int32_t* q_sizes, const int32_t* k_sizes, int64_t bh_q,
                                                  int64_t bh_kv, int64_t s, int32_t d, int32_t qn, int32_t kn,
                                                  float scale, const int32_t* q_index, const int32_t* k_index,
                                                  void* out, float* lse, hipStream_t stream) {
  SPR_REQUIRE(bh_q >= 0 && bh_kv >= 1 && s >= 0 && qn >= 1 && kn >= 1, "spr_block_sparse_attention_noalloc: bad size");
  if (bh_q == 0 || s == 0) return SPR_OK;
  SPR_REQUIRE(kn <= 16384 && qn <= TO_MAX_QN && bh_kv <= 65535, "spr_block_sparse_attention_noalloc: bad plan size");
  const size_t need = spr_block_sparse_attention_workspace(bh_kv, qn, kn);
  if (need > NOALLOC_PLAN_BYTES) {
    spr_set_error("spr_block_sparse_attention_noalloc: the plan for bh_kv=%lld qn=%d kn=%d needs %zu bytes, more "
                  "than the %zu-byte fixed plan array; use spr_block_sparse_attention with a workspace",
                  (long long)bh_kv, qn, kn, need, NOALLOC_PLAN_BYTES);
    return SPR_EWORKSPACE;
  }
  void* plan = nullptr;
  const int st = noalloc_scratch_addr(&plan);
  if (st != SPR_OK) return st;
  return spr_block_sparse_attention(q, k, v, map, q_sizes, k_sizes, bh_q, bh_kv, s, d, qn, kn, scale, q_index,
                                    k_index, out, lse, plan, need, stream);
}
