// layout.hip -- the tiled arena's backward tables built on the device.
//
// The physical arena (dst-sorted slabs, units renumbered busiest source
// first) is laid out with the structural entry points (compaction, stable
// radix sort, gathers); these kernels add what the tiled backward needs per
// bucket: every tile's (source, position) order, its (tile, source) groups
// and their descriptors, the hot ranks and the cold slots' region counts.
// One workgroup per tile sorts the tile's keys in LDS, so the whole
// transpose costs two passes over FROM_ID instead of a global sort by
// (tile, source). The tables equal the host build's (plastax_amd/_layout.py)
// entry for entry.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/plastax_hip.h"
#include "px_common.h"

using plx_detail::check_launch;
using plx_detail::fail;

namespace {

constexpr int kTB = 512;          // threads per tile workgroup
constexpr int kTileMax = 4096;    // positions per tile at most
constexpr int kPerT = kTileMax / kTB;
constexpr uint32_t kStart = 0x8000u;

// Sorts keys[0, kTileMax) ascending (bitonic; every thread takes part).
template <typename K>
__device__ void bitonic4096(K* keys) {
  for (int k = 2; k <= kTileMax; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < kTileMax; i += kTB) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const K a = keys[i], b = keys[ixj];
          const bool up = (i & k) == 0;
          if ((a > b) == up) {
            keys[i] = b;
            keys[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Exclusive scan of one int per thread over the workgroup (wave prefix
// sums, then the waves' totals); *total gets the sum.
__device__ int block_scan(int v, int* lds, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) lds[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < kTB / 64; ++w) {
      const int t = lds[w];
      lds[w] = run;
      run += t;
    }
    lds[kTB / 64] = run;
  }
  __syncthreads();
  const int out = lds[wave] + x - v;
  *total = lds[kTB / 64];
  __syncthreads();
  return out;
}

// The tile's live positions' keys (source << 12 | position in the tile, in
// 64 bits, so any int32 source id fits), sorted; n = their number. A tile
// spanning more than kTileMax positions breaks the caller's contract: its
// first kTileMax positions are sorted (every LDS access stays in bounds) and
// *over is set.
__device__ int load_sorted(const plx_tile_build_desc& d, int t, uint64_t* keys, bool* over) {
  const int p0 = d.tile_pos[t];
  const int span = max(0, min(d.tile_pos[t + 1], d.live) - p0);
  *over = span > kTileMax;
  const int n = min(span, kTileMax);
  for (int i = threadIdx.x; i < kTileMax; i += kTB)
    keys[i] = i < n ? (static_cast<uint64_t>(static_cast<uint32_t>(d.src[p0 + i])) << 12) | static_cast<uint64_t>(i)
                    : ~0ull;
  __syncthreads();
  bitonic4096(keys);
  return n;
}

__device__ __forceinline__ uint32_t key_src(uint64_t k) { return static_cast<uint32_t>(k >> 12); }

// Pass 0: groups per tile, and every group's source counted in presence.
// A tile longer than kTileMax positions reports -1 groups (the host reads
// the counts and refuses the layout).
__global__ __launch_bounds__(kTB) void k_tile_count(plx_tile_build_desc d) {
  __shared__ uint64_t keys[kTileMax];
  __shared__ int scan_lds[kTB / 64 + 1];
  const int t = blockIdx.x;
  bool over = false;
  const int n = load_sorted(d, t, keys, &over);
  int mine = 0;
  for (int k = 0; k < kPerT; ++k) {
    const int i = threadIdx.x * kPerT + k;
    if (i < n && (i == 0 || key_src(keys[i]) != key_src(keys[i - 1]))) {
      ++mine;
      atomicAdd(d.presence + key_src(keys[i]), 1);
    }
  }
  int total = 0;
  block_scan(mine, scan_lds, &total);
  if (threadIdx.x == 0) d.ngroups[t] = over ? -1 : total;
}

// Pass 1: the tile's tables.
__global__ __launch_bounds__(kTB) void k_tile_tables(plx_tile_build_desc d) {
  __shared__ uint64_t keys[kTileMax];
  __shared__ uint32_t gkey[kTileMax];
  __shared__ uint16_t gstart[kTileMax + 1];  // ranks 0..kTileMax; the workgroup stays within 64 KiB of LDS
  __shared__ int scan_lds[kTB / 64 + 1];
  __shared__ int counts[2 + 8];
  const int t = blockIdx.x;
  const int p0 = d.tile_pos[t];
  bool over = false;
  const int n = load_sorted(d, t, keys, &over);
  const uint32_t hb = static_cast<uint32_t>(d.hot_base), he = hb + static_cast<uint32_t>(d.nhot);
  if (threadIdx.x < 10) counts[threadIdx.x] = 0;
  // Group starts of this thread's consecutive ranks, then their indices.
  bool st[kPerT];
  int mine = 0;
  for (int k = 0; k < kPerT; ++k) {
    const int i = threadIdx.x * kPerT + k;
    st[k] = i < n && (i == 0 || key_src(keys[i]) != key_src(keys[i - 1]));
    mine += st[k];
  }
  int ng = 0;
  int g = block_scan(mine, scan_lds, &ng);
  int hlo = 0, hcnt = 0;
  int rc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int k = 0; k < kPerT; ++k) {
    const int i = threadIdx.x * kPerT + k;
    if (i >= n) break;
    const uint32_t src = key_src(keys[i]);
    const int pos = p0 + static_cast<int>(keys[i] & 0xFFFu);
    d.sorted_rank[pos] = static_cast<uint16_t>(static_cast<uint32_t>(i) | (st[k] ? kStart : 0u));
    if (st[k]) gstart[g++] = static_cast<uint16_t>(i);
    if (src < hb)
      ++hlo;
    else if (src < he)
      ++hcnt;
    if (src < hb || src >= he) ++rc[d.region[src] & 7];
  }
  if (threadIdx.x == 0) gstart[ng] = static_cast<uint16_t>(n);
  atomicAdd(&counts[0], hlo);
  atomicAdd(&counts[1], hcnt);
  for (int x = 0; x < 8; ++x)
    if (rc[x]) atomicAdd(&counts[2 + x], rc[x]);
  __syncthreads();
  // Groups in source order: their source, first rank and tile; and the
  // descriptor keys (longest first, then source order).
  const int g0 = d.grp_off[t];
  for (int q = threadIdx.x; q < kTileMax; q += kTB) {
    if (q < ng) {
      const int s0 = gstart[q], len = gstart[q + 1] - s0;
      d.g_src[g0 + q] = static_cast<int32_t>(key_src(keys[s0]));
      d.g_st[g0 + q] = s0;
      d.g_tile[g0 + q] = t;
      gkey[q] = (static_cast<uint32_t>(kTileMax - len) << 12) | static_cast<uint32_t>(q);
    } else {
      gkey[q] = 0xFFFFFFFFu;
    }
  }
  __syncthreads();
  bitonic4096(gkey);
  for (int q = threadIdx.x; q < ng; q += kTB) {
    const int gi = static_cast<int>(gkey[q] & 0xFFFu);
    const int s0 = gstart[gi], len = gstart[gi + 1] - s0;
    d.grp[g0 + q] = static_cast<uint16_t>(static_cast<uint32_t>(s0) | (static_cast<uint32_t>(min(len, 15)) << 12));
  }
  if (threadIdx.x < 2) d.hl[2 * t + threadIdx.x] = counts[threadIdx.x];
  if (threadIdx.x < 8) d.cnt[8 * t + threadIdx.x] = counts[2 + threadIdx.x];
}

__global__ void k_cold_slots(int64_t n, const int32_t* n_dev, const int32_t* cold, const int32_t* g_src,
                             const int32_t* g_st, const int32_t* g_tile, const int32_t* hl, const int32_t* off,
                             const int8_t* region, const int32_t* sb_of_tile, int32_t* cold_idx,
                             uint16_t* cold_sb) {
  const int64_t m = n_dev ? *n_dev : n;
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; k < m;
       k += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t g = cold[k];
    const int32_t t = g_tile[g], s0 = g_st[g];
    const int32_t hlo = hl[2 * t], hcnt = hl[2 * t + 1];
    const int32_t c = s0 >= hlo + hcnt ? s0 - hcnt : s0;
    cold_idx[k] = off[8 * t + (region[g_src[g]] & 7)] + c;
    cold_sb[k] = static_cast<uint16_t>(sb_of_tile[t]);
  }
}

// Runs of equal ids among a wave's consecutive lanes add once, from their
// first lane (the logical buckets are source-major and the slabs
// destination-sorted, so most ids repeat across neighbouring positions and
// a plain per-position atomic would serialise on them).
__global__ void k_count_ids(int64_t n, const int32_t* ids, const uint8_t* skip, int32_t nbins, int32_t* counts) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * blockDim.x; base < n; base += stride) {
    const int64_t p = base + threadIdx.x;
    int32_t u = -1;
    if (p < n && !(skip && skip[p])) {
      u = ids[p];
      if (u < 0 || u >= nbins) u = -1;
    }
    const int32_t prev = __shfl_up(u, 1, 64);
    const bool head = lane == 0 || prev != u;
    const uint64_t heads = __ballot(head);
    if (head && u >= 0) {
      const uint64_t after = lane == 63 ? 0ull : (heads >> (lane + 1));
      const int len = after ? __builtin_ctzll(after) + 1 : 64 - lane;
      atomicAdd(counts + u, len);
    }
  }
}

__global__ void k_copy_to_slots(int64_t n, const int32_t* n_dev, const int32_t* pos, const int32_t* slot,
                                const void* src, void* dst, int64_t dst_len, int32_t bytes) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n || (n_dev && i >= *n_dev)) return;
  const int32_t p = pos[i];
  const int64_t s = slot[p];
  if (s < 0 || s >= dst_len) return;
  if (bytes == 1) static_cast<uint8_t*>(dst)[s] = static_cast<const uint8_t*>(src)[p];
  else static_cast<uint32_t*>(dst)[s] = static_cast<const uint32_t*>(src)[p];
}

// The (key1, key2) of id `id` of a merge side, as one 64-bit unsigned key;
// ids are clamped into [0, id_limit) for the reads.
__device__ __forceinline__ uint64_t merge_key(const plx_merge_side& s, int64_t id) {
  id = id < 0 ? 0 : (id >= s.id_limit ? s.id_limit - 1 : id);
  const uint32_t k1 = static_cast<uint32_t>(s.key1[id]);
  const uint32_t k2 = s.key2 ? static_cast<uint32_t>(s.key2[id]) : static_cast<uint32_t>(id);
  return (static_cast<uint64_t>(k1) << 32) | k2;
}

// A side's element count: n, or *n_dev (at most n) when the count is on the
// device.
__device__ __forceinline__ int64_t side_count(const plx_merge_side& s) {
  if (!s.n_dev) return s.n;
  const int64_t c = *s.n_dev;
  return c < 0 ? 0 : (c < s.n ? c : s.n);
}

// The number of the first n elements of `s` whose key is below `key`
// (or_equal: at most `key`): a binary search over the side's sorted ids.
__device__ __forceinline__ int64_t merge_count(const plx_merge_side& s, int64_t n, uint64_t key, bool or_equal) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    const uint64_t k = merge_key(s, s.ids[mid]);
    if (k < key || (or_equal && k == key)) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

__device__ __forceinline__ void merge_put(const plx_merge_desc& d, const plx_merge_side& s, int64_t r,
                                          int32_t code, int64_t id) {
  if (d.order) d.order[r] = code;
  if (s.map && id >= 0 && id < s.id_limit) s.map[id] = static_cast<int32_t>(r + d.offset);
}

constexpr int kMergeBlock = 256;
constexpr int kMergeStaged = 2048;  // b keys staged in LDS (16 KiB); a longer b is searched in global memory

// The number of the n keys of `keys` (ascending, in LDS) below `key`.
__device__ __forceinline__ int64_t lds_count(const uint64_t* keys, int64_t n, uint64_t key) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

constexpr int kMergePer = 4;  // elements per thread: their loads are in flight together

// One thread per element i of a (a is the long side: the survivors), four
// per thread (element i = block * 1024 + k * 256 + lane). With c(i) the
// number of b elements below a's i-th key (a first on ties), a_i lands at
// i + c(i), and b_j for c(i-1) <= j < c(i) lands just before it, at j + i;
// the last element's thread places the b elements after every a. Each
// thread searches only b (its keys staged in LDS) and takes c(i-1) from the
// block's table. With a empty, b_j lands at j.
__global__ __launch_bounds__(kMergeBlock) void k_merge_index(plx_merge_desc d) {
  __shared__ uint64_t bkey[kMergeStaged];
  __shared__ int64_t cnt[kMergeBlock * kMergePer];
  const int64_t na = side_count(d.a), nb = side_count(d.b);
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kMergeBlock * kMergePer;
  if (na == 0) {  // uniform over the grid
    for (int k = 0; k < kMergePer; ++k) {
      const int64_t t = first + k * kMergeBlock + threadIdx.x;
      if (t < nb) merge_put(d, d.b, t, static_cast<int32_t>(-1 - t), d.b.ids[t]);
    }
    return;
  }
  if (first >= na) return;  // uniform over the workgroup: the grid is sized for the sides' maxima
  const bool staged = nb <= kMergeStaged;
  if (staged)
    for (int64_t j = threadIdx.x; j < nb; j += kMergeBlock) bkey[j] = merge_key(d.b, d.b.ids[j]);
  int64_t id[kMergePer];
  uint64_t key[kMergePer];
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) {
    const int64_t t = first + k * kMergeBlock + threadIdx.x;
    id[k] = t < na ? d.a.ids[t] : 0;
  }
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) key[k] = merge_key(d.a, id[k]);
  __syncthreads();
  int64_t c[kMergePer];
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) {
    c[k] = staged ? lds_count(bkey, nb, key[k]) : merge_count(d.b, nb, key[k], false);
    cnt[k * kMergeBlock + threadIdx.x] = c[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) {
    const int e = k * kMergeBlock + threadIdx.x;  // the element's index in the block
    const int64_t t = first + e;
    if (t >= na) break;
    merge_put(d, d.a, t + c[k], static_cast<int32_t>(id[k]), id[k]);
    int64_t c0 = 0;
    if (e > 0) {
      c0 = cnt[e - 1];
    } else if (t > 0) {
      const uint64_t kp = merge_key(d.a, d.a.ids[t - 1]);
      c0 = staged ? lds_count(bkey, nb, kp) : merge_count(d.b, nb, kp, false);
    }
    for (int64_t j = c0; j < c[k]; ++j) merge_put(d, d.b, j + t, static_cast<int32_t>(-1 - j), d.b.ids[j]);
    if (t == na - 1)
      for (int64_t j = c[k]; j < nb; ++j) merge_put(d, d.b, j + na, static_cast<int32_t>(-1 - j), d.b.ids[j]);
  }
}

// Four ranks per thread (rank = block * 1024 + k * 256 + lane); each
// column's element comes from a (by the id in `order`) or from b (by the id
// in b_ids). NC columns, a compile-time count, so the values stay in
// registers and every load is issued before any store.
template <int NC>
__global__ __launch_bounds__(256) void k_merge_gather(plx_merge_gather_desc d) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 * kMergePer;
  // ranks below cnt are gathered; with n_dev, ranks [cnt, n) get the
  // columns' fill values
  int64_t cnt = d.n;
  if (d.n_dev) {
    const int64_t c = *d.n_dev;
    cnt = c < 0 ? 0 : (c < d.n ? c : d.n);
  }
  bool ok[kMergePer], from_a[kMergePer];
  int64_t at[kMergePer];
  int32_t id[kMergePer];
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) {
    const int64_t r = first + k * 256 + threadIdx.x;
    ok[k] = r < cnt;
    const int32_t o = ok[k] ? d.order[r] : 0;
    // Every index is clamped into its array (a malformed order reads a
    // wrong element rather than outside the buffers).
    from_a[k] = o >= 0 || d.nb == 0;
    id[k] = 0;
    if (from_a[k]) {
      at[k] = o < 0 ? 0 : (o < d.a_limit ? o : d.a_limit - 1);
    } else {
      int64_t j = -1 - static_cast<int64_t>(o);
      j = j < d.nb ? j : d.nb - 1;
      id[k] = d.b_ids[j];
      at[k] = id[k] < 0 ? 0 : (id[k] >= d.b_limit ? d.b_limit - 1 : id[k]);
    }
  }
  uint32_t v[NC][kMergePer];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const plx_merge_col& col = d.cols[c];
#pragma unroll
    for (int k = 0; k < kMergePer; ++k) {
      const void* src = from_a[k] ? col.a : col.b;
      v[c][k] = !ok[k] ? 0u
                : !src    ? static_cast<uint32_t>(id[k])
                : col.bytes == 1 ? static_cast<uint32_t>(static_cast<const uint8_t*>(src)[at[k]])
                                 : static_cast<const uint32_t*>(src)[at[k]];
    }
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const plx_merge_col& col = d.cols[c];
#pragma unroll
    for (int k = 0; k < kMergePer; ++k) {
      const int64_t r = first + k * 256 + threadIdx.x;
      if (r >= d.n) continue;
      const uint32_t x = ok[k] ? v[c][k] : col.fill;
      if (col.bytes == 1) static_cast<uint8_t*>(col.out)[r] = static_cast<uint8_t>(x);
      else static_cast<uint32_t*>(col.out)[r] = x;
    }
  }
}

template <int NC>
void launch_merge_gather(const plx_merge_gather_desc& d, hipStream_t s) {
  if (d.ncols == NC) {
    hipLaunchKernelGGL(k_merge_gather<NC>, dim3(static_cast<unsigned>((d.n + 256 * kMergePer - 1) / (256 * kMergePer))),
                       dim3(256), 0, s, d);
    return;
  }
  if constexpr (NC < PLX_MERGE_MAX_COLS) launch_merge_gather<NC + 1>(d, s);
}

// Four entries per thread, their loads in flight together.
__global__ __launch_bounds__(256) void k_remap_i32(int64_t n, const int32_t* idx, int64_t off, int64_t map_len,
                                                   const int32_t* map, int32_t* out, uint8_t* live) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 * kMergePer;
  int64_t p[kMergePer];
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) {
    const int64_t j = first + k * 256 + threadIdx.x;
    p[k] = j < n ? static_cast<int64_t>(idx[j]) - off : -1;
  }
  int32_t m[kMergePer];
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) m[k] = (p[k] >= 0 && p[k] < map_len) ? map[p[k]] : -1;
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) {
    const int64_t j = first + k * 256 + threadIdx.x;
    if (j >= n) break;
    out[j] = m[k];
    live[j] = m[k] >= 0;
  }
}

// plx_remap_merged: the dropped positions and the inserted elements' ranks
// among the survivors staged in LDS (both at most PLX_REMAP_LDS_MAX, else
// the map is read), then two binary searches per entry.
__global__ __launch_bounds__(256) void k_remap_merged(int64_t n, const int32_t* idx, int64_t off, int64_t map_len,
                                                     const int32_t* map, const int32_t* dropped,
                                                     const int32_t* ndropped, const int32_t* ins,
                                                     const int32_t* nins, int64_t ins_len,
                                                     const int32_t* new_pos, int32_t* out, uint8_t* live) {
  __shared__ int32_t sk[PLX_REMAP_LDS_MAX], sr[PLX_REMAP_LDS_MAX];
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 * kMergePer;
  // (the counts clamped to their lists' lengths)
  const int nk = static_cast<int>(min(static_cast<int64_t>(max(*ndropped, 0)), map_len));
  const int ni = static_cast<int>(min(static_cast<int64_t>(max(*nins, 0)), ins_len));
  const bool staged = nk <= PLX_REMAP_LDS_MAX && ni <= PLX_REMAP_LDS_MAX;  // uniform
  if (staged) {
    for (int i = threadIdx.x; i < nk; i += 256) sk[i] = dropped[i];
    // the number of survivors placed before inserted element i
    for (int i = threadIdx.x; i < ni; i += 256) sr[i] = static_cast<int32_t>(new_pos[ins[i]] - off - i);
  }
  __syncthreads();
  int64_t p[kMergePer];
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) {
    const int64_t j = first + k * 256 + threadIdx.x;
    p[k] = j < n ? static_cast<int64_t>(idx[j]) - off : -1;
  }
  int32_t m[kMergePer];
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) {
    const bool in = p[k] >= 0 && p[k] < map_len;
    if (!in) {
      m[k] = -1;
    } else if (!staged) {
      m[k] = map[p[k]];
    } else {
      const int32_t q = static_cast<int32_t>(p[k]);
      int lo = 0, hi = nk;  // the dropped positions below q
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sk[mid] < q) lo = mid + 1; else hi = mid;
      }
      if (lo < nk && sk[lo] == q) {
        m[k] = -1;
      } else {
        const int32_t sv = q - lo;  // the survivor's rank
        int a = 0, b = ni;          // the inserted elements with sr <= sv
        while (a < b) {
          const int mid = (a + b) >> 1;
          if (sr[mid] <= sv) a = mid + 1; else b = mid;
        }
        m[k] = static_cast<int32_t>(sv + a + off);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kMergePer; ++k) {
    const int64_t j = first + k * 256 + threadIdx.x;
    if (j >= n) break;
    out[j] = m[k];
    live[j] = m[k] >= 0;
  }
}

unsigned grid_of(int64_t n, int block) {
  const int64_t g = (n + block - 1) / block;
  return static_cast<unsigned>(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

// plx_claimed_split: one workgroup per bucket keeps the listed slots in its
// range (less its start) and writes the first min(count, region) of them in
// ascending order. The slots are distinct, so up to kSplitRank listed
// entries each one's rank is the number of smaller ones (a broadcast LDS
// loop); longer lists sort in LDS (bitonic over the next power of two;
// absent entries sort last).
static_assert(PLX_CLAIMED_SPLIT_MAX == kTileMax, "the split sorts one LDS tile");
constexpr int kSplitRank = 1024;
__global__ __launch_bounds__(kTB) void k_claimed_split(int64_t cap, const int32_t* n_dev, const int32_t* list,
                                                      const int64_t* offs, int64_t region, int32_t* out,
                                                      int32_t* counts) {
  __shared__ uint32_t keys[kTileMax];
  __shared__ int kept;
  const int b = static_cast<int>(blockIdx.x);
  const int64_t lo = offs[b], hi = offs[b + 1];
  int64_t nl = *n_dev;
  const int n = static_cast<int>(nl < 0 ? 0 : (nl < cap ? nl : cap));
  int p2 = 1;
  while (p2 < n) p2 <<= 1;
  if (threadIdx.x == 0) kept = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < p2; i += kTB) {
    uint32_t k = 0xFFFFFFFFu;
    if (i < n) {
      const int64_t v = list[i];
      if (v >= lo && v < hi) {
        k = static_cast<uint32_t>(v - lo);
        atomicAdd(&kept, 1);
      }
    }
    keys[i] = k;
  }
  __syncthreads();
  const int c = kept;
  int32_t* o = out + static_cast<int64_t>(b) * region;
  if (n <= kSplitRank) {
    for (int i = threadIdx.x; i < n; i += kTB) {
      const uint32_t k = keys[i];
      if (k == 0xFFFFFFFFu) continue;
      int r = 0;
      for (int j = 0; j < n; ++j) r += keys[j] < k ? 1 : 0;
      if (r < region) o[r] = static_cast<int32_t>(k);
    }
  } else {
    for (int k = 2; k <= p2; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = threadIdx.x; i < p2; i += kTB) {
          const int ixj = i ^ j;
          if (ixj > i) {
            const uint32_t x = keys[i], y = keys[ixj];
            const bool up = (i & k) == 0;
            if ((x > y) == up) {
              keys[i] = y;
              keys[ixj] = x;
            }
          }
        }
        __syncthreads();
      }
    }
    for (int64_t i = threadIdx.x; i < c && i < region; i += kTB) o[i] = static_cast<int32_t>(keys[i]);
  }
  if (threadIdx.x == 0) counts[b] = c;
}

}  // namespace

extern "C" {

int plx_tile_build(const plx_tile_build_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_tile_build: null descriptor");
  if (d->ntiles < 0 || d->live < 0) return fail(PLX_ERR_INVALID, "plx_tile_build: negative sizes");
  if (d->ntiles == 0) return PLX_OK;
  if (!d->tile_pos || (d->live > 0 && !d->src)) return fail(PLX_ERR_INVALID, "plx_tile_build: null column");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (d->pass == 0) {
    if (!d->ngroups || !d->presence) return fail(PLX_ERR_INVALID, "plx_tile_build: pass 0 outputs missing");
    hipLaunchKernelGGL(k_tile_count, dim3(d->ntiles), dim3(kTB), 0, s, *d);
  } else if (d->pass == 1) {
    if (!d->grp_off || !d->region || !d->sorted_rank || !d->grp || !d->g_src || !d->g_st || !d->g_tile || !d->hl ||
        !d->cnt)
      return fail(PLX_ERR_INVALID, "plx_tile_build: pass 1 tables missing");
    if (d->nhot < 0 || d->hot_base < 0) return fail(PLX_ERR_INVALID, "plx_tile_build: bad hot range");
    hipLaunchKernelGGL(k_tile_tables, dim3(d->ntiles), dim3(kTB), 0, s, *d);
  } else {
    return fail(PLX_ERR_INVALID, "plx_tile_build: pass must be 0 or 1");
  }
  return check_launch("plx_tile_build");
}

int plx_cold_slots(int64_t n, const int32_t* n_dev, const int32_t* cold, const int32_t* g_src, const int32_t* g_st,
                   const int32_t* g_tile, const int32_t* hl, const int32_t* off, const int8_t* region,
                   const int32_t* sb_of_tile, int32_t* cold_idx, uint16_t* cold_sb, void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_cold_slots: negative n");
  if (n == 0) return PLX_OK;
  if (!cold || !g_src || !g_st || !g_tile || !hl || !off || !region || !sb_of_tile || !cold_idx || !cold_sb)
    return fail(PLX_ERR_INVALID, "plx_cold_slots: null pointer");
  hipLaunchKernelGGL(k_cold_slots, dim3(grid_of(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream), n, n_dev,
                     cold, g_src, g_st, g_tile, hl, off, region, sb_of_tile, cold_idx, cold_sb);
  return check_launch("plx_cold_slots");
}

int plx_copy_to_slots(int64_t n, const int32_t* n_dev, const int32_t* pos, const int32_t* slot, const void* src,
                      void* dst, int64_t dst_len, int32_t bytes, void* stream) {
  if (n < 0 || dst_len < 0) return fail(PLX_ERR_INVALID, "plx_copy_to_slots: negative size");
  if (bytes != 1 && bytes != 4) return fail(PLX_ERR_INVALID, "plx_copy_to_slots: bytes must be 1 or 4");
  if (n == 0) return PLX_OK;
  if (!pos || !slot || !src || !dst) return fail(PLX_ERR_INVALID, "plx_copy_to_slots: null pointer");
  hipLaunchKernelGGL(k_copy_to_slots, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), n, n_dev, pos, slot, src, dst, dst_len, bytes);
  return check_launch("plx_copy_to_slots");
}

static bool merge_side_ok(const plx_merge_side& s) {
  if (s.n < 0 || s.id_limit < 0) return false;
  if (s.n == 0) return true;
  return s.ids && s.key1 && s.id_limit > 0;
}

int plx_merge_index(const plx_merge_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_merge_index: null descriptor");
  if (!merge_side_ok(d->a) || !merge_side_ok(d->b)) return fail(PLX_ERR_INVALID, "plx_merge_index: bad side");
  const int64_t n = d->a.n + d->b.n;
  if (n > INT32_MAX || d->offset < 0 || d->offset + n > INT32_MAX)
    return fail(PLX_ERR_INVALID, "plx_merge_index: ranks exceed int32");
  if (n == 0) return PLX_OK;
  // one thread per element of a, or of b when a is empty (counts on the
  // device: sized for the larger maximum, the rest of the grid exits)
  const int64_t elems = d->a.n > d->b.n ? d->a.n : d->b.n;
  const int64_t per_block = static_cast<int64_t>(kMergeBlock) * kMergePer;
  hipLaunchKernelGGL(k_merge_index, dim3(static_cast<unsigned>((elems + per_block - 1) / per_block)),
                     dim3(kMergeBlock), 0, static_cast<hipStream_t>(stream), *d);
  return check_launch("plx_merge_index");
}

int plx_merge_gather(const plx_merge_gather_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_merge_gather: null descriptor");
  if (d->n < 0 || d->nb < 0 || d->ncols < 0 || d->ncols > PLX_MERGE_MAX_COLS)
    return fail(PLX_ERR_INVALID, "plx_merge_gather: bad sizes");
  if (d->n == 0 || d->ncols == 0) return PLX_OK;
  if (!d->order || d->a_limit <= 0 || (d->nb > 0 && (!d->b_ids || d->b_limit <= 0)))
    return fail(PLX_ERR_INVALID, "plx_merge_gather: null order or empty side");
  for (int k = 0; k < d->ncols; ++k) {
    const plx_merge_col& c = d->cols[k];
    if (!c.a || !c.out || (c.bytes != 1 && c.bytes != 4))
      return fail(PLX_ERR_INVALID, "plx_merge_gather: bad column");
  }
  launch_merge_gather<1>(*d, static_cast<hipStream_t>(stream));
  return check_launch("plx_merge_gather");
}

int plx_remap_i32(int64_t n, const int32_t* idx, int64_t off, int64_t map_len, const int32_t* map, int32_t* out,
                  uint8_t* live, void* stream) {
  if (n < 0 || map_len < 0) return fail(PLX_ERR_INVALID, "plx_remap_i32: negative size");
  if (n == 0) return PLX_OK;
  if (!idx || !map || !out || !live) return fail(PLX_ERR_INVALID, "plx_remap_i32: null pointer");
  hipLaunchKernelGGL(k_remap_i32, dim3(static_cast<unsigned>((n + 256 * kMergePer - 1) / (256 * kMergePer))),
                     dim3(256), 0,
                     static_cast<hipStream_t>(stream), n, idx, off, map_len, map, out, live);
  return check_launch("plx_remap_i32");
}

int plx_count_ids(int64_t n, const int32_t* ids, const uint8_t* skip, int32_t nbins, int32_t* counts, void* stream) {
  if (n < 0 || nbins < 0) return fail(PLX_ERR_INVALID, "plx_count_ids: negative size");
  if (n == 0) return PLX_OK;
  if (!ids || !counts) return fail(PLX_ERR_INVALID, "plx_count_ids: null pointer");
  hipLaunchKernelGGL(k_count_ids, dim3(grid_of(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream), n, ids, skip,
                     nbins, counts);
  return check_launch("plx_count_ids");
}

int plx_claimed_split(int64_t cap, const int32_t* n_dev, const int32_t* list, int32_t nb, const int64_t* offs,
                      int64_t region, int32_t* out, int32_t* counts, void* stream) {
  if (cap < 0 || nb < 0 || region < 0) return fail(PLX_ERR_INVALID, "plx_claimed_split: negative size");
  if (cap > PLX_CLAIMED_SPLIT_MAX) return fail(PLX_ERR_UNSUPPORTED, "plx_claimed_split: cap above PLX_CLAIMED_SPLIT_MAX");
  if (nb == 0) return PLX_OK;
  if (!n_dev || !offs || !counts || (cap > 0 && !list) || (region > 0 && !out))
    return fail(PLX_ERR_INVALID, "plx_claimed_split: null pointer");
  hipLaunchKernelGGL(k_claimed_split, dim3(static_cast<unsigned>(nb)), dim3(kTB), 0, static_cast<hipStream_t>(stream),
                     cap, n_dev, list, offs, region, out, counts);
  return check_launch("plx_claimed_split");
}

int plx_remap_merged(int64_t n, const int32_t* idx, int64_t off, int64_t map_len, const int32_t* map,
                     const int32_t* dropped, const int32_t* ndropped, const int32_t* ins, const int32_t* nins,
                     int64_t ins_len, const int32_t* new_pos, int32_t* out, uint8_t* live, void* stream) {
  if (n < 0 || map_len < 0 || ins_len < 0) return fail(PLX_ERR_INVALID, "plx_remap_merged: negative size");
  if (n == 0) return PLX_OK;
  if (!idx || !map || !dropped || !ndropped || !ins || !nins || !new_pos || !out || !live)
    return fail(PLX_ERR_INVALID, "plx_remap_merged: null pointer");
  hipLaunchKernelGGL(k_remap_merged, dim3(static_cast<unsigned>((n + 256 * kMergePer - 1) / (256 * kMergePer))),
                     dim3(256), 0, static_cast<hipStream_t>(stream), n, idx, off, map_len, map, dropped, ndropped,
                     ins, nins, ins_len, new_pos, out, live);
  return check_launch("plx_remap_merged");
}

}  // extern "C"
