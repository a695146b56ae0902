// structural.hip -- gfx950 kernels of the structural phases (PruneConn and
// add_conn growth) and the C ABI declared in include/plastax_hip.h.
//
// These phases are integer / ordering work over candidate lists and the
// logical arena: evaluate a traced callback once per site, compact the
// survivors in order, sort them into the library's total order, select the
// first k per source level and claim free slots in order. Every result is an
// exact function of its inputs (integer atomics only count; no float
// atomics), so the device reproduces the CPU restatement bit for bit.
//
// Building blocks:
//  - site programs: a register interpreter over 32-bit float/int/uint/bool
//    values, one thread per site, with the counter-based Philox stream of
//    rng.py (no device state);
//  - ordered compaction and exclusive scans: per-chunk counts (2048
//    elements per 256-lane workgroup), one workgroup scanning the chunk
//    totals, then a chunk pass that ranks with wave ballots and LDS;
//  - stable LSD radix sort: 8-bit digits over 4096-element tiles, a
//    digit-major histogram per tile, its scan, and a scatter that ranks each
//    round of 256 keys with 8 wave ballots (peers with the same digit) plus
//    per-wave LDS counts.
#include <hip/hip_runtime.h>

#include <hip/hiprtc.h>

#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/plastax_hip.h"
#include "px_common.h"
#include "px_math.h"
#include "px_site.h"

using plx_detail::check_launch;
using plx_detail::fail;

namespace {

constexpr int kBlock = 256;          // lanes per workgroup (4 waves of 64)
static_assert(kBlock == kSiteBlock, "site programs are launched with kSiteBlock lanes");
constexpr int kWaves = kBlock / 64;
constexpr int kChunk = kBlock * 8;   // elements per scan / compaction chunk
constexpr int kTile = kBlock * 16;   // elements per radix tile
constexpr int kScanLanes = 1024;     // the single-workgroup scan

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return lane ? (~0ull >> (64 - lane)) : 0ull;
}

// Exclusive scan across a workgroup of BLOCK lanes; *total gets the sum.
// lds: BLOCK / 64 + 1 ints. Every lane must call it.
template <int BLOCK>
__device__ __forceinline__ int block_exclusive_scan(int v, int* lds, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) lds[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < BLOCK / 64; ++w) {
      const int t = lds[w];
      lds[w] = run;
      run += t;
    }
    lds[BLOCK / 64] = run;
  }
  __syncthreads();
  const int out = x - v + lds[wave];
  *total = lds[BLOCK / 64];
  __syncthreads();
  return out;
}

// ---------------------------------------------------------------------------
// Flags, chunk sums and the scans.
// ---------------------------------------------------------------------------

// The R values a thread reads of the chunk at `base` (positions base + r *
// kBlock + threadIdx.x; base < n): mode < 0 the int32 values of `in`, else
// the flags of the compaction mode (0 or 1); positions at or past n give 0.
// The mode is uniform, so each case is straight-line code: every load is
// issued (past n at the last position) before any is used, one memory
// latency per chunk instead of one per round.
template <int R>
__device__ __forceinline__ void chunk_values(int32_t mode, const void* in, int64_t base, int64_t n, int* v) {
  int64_t q[R];
  bool ok[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t p = base + r * kBlock + threadIdx.x;
    ok[r] = p < n;
    q[r] = ok[r] ? p : n - 1;
  }
  if (mode == PLX_FLAG_U8 || mode == PLX_FLAG_U8_ZERO) {
    uint32_t b[R];
#pragma unroll
    for (int r = 0; r < R; ++r) b[r] = static_cast<const uint8_t*>(in)[q[r]];
    const bool want = mode == PLX_FLAG_U8;
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = ok[r] && ((b[r] != 0u) == want);
  } else if (mode == PLX_FLAG_FINITE) {
    uint32_t b[R];
#pragma unroll
    for (int r = 0; r < R; ++r) b[r] = static_cast<const uint32_t*>(in)[q[r]];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = ok[r] && (b[r] & 0x7F800000u) != 0x7F800000u;
  } else {
    int b[R];
#pragma unroll
    for (int r = 0; r < R; ++r) b[r] = static_cast<const int32_t*>(in)[q[r]];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = !ok[r] ? 0 : (mode < 0 ? b[r] : (b[r] != 0));
  }
}

// mode < 0: the values of `in` (a scan); else the flags (a compaction).
__global__ void k_chunk_sums(int64_t n_max, const int32_t* n_dev, int32_t mode, const void* in,
                             int32_t* sums) {
  __shared__ int lds[kWaves + 1];
  const int64_t n = live_count(n_max, n_dev);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
  if (base >= n) {  // a chunk past the count sums to 0 (uniform over the workgroup)
    if (threadIdx.x == 0) sums[blockIdx.x] = 0;
    return;
  }
  constexpr int R = kChunk / kBlock;
  int v[R];
  chunk_values<R>(mode, in, base, n, v);
  int acc = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) acc += v[r];
  int total;
  block_exclusive_scan<kBlock>(acc, lds, &total);
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// One workgroup: exclusive scan of sums[0, m) in place, 1024 consecutive
// entries per round (coalesced); total (optional). Used for the chunk totals
// of the multi-workgroup scans, so m stays small.
__global__ void k_scan_single(int64_t m, int32_t* sums, int32_t* total) {
  __shared__ int lds[kScanLanes / 64 + 1];
  int run = 0;
  for (int64_t base = 0; base < m; base += kScanLanes) {
    const int64_t i = base + threadIdx.x;
    const int v = i < m ? sums[i] : 0;
    int all;
    const int ex = block_exclusive_scan<kScanLanes>(v, lds, &all);
    if (i < m) sums[i] = run + ex;
    run += all;
  }
  if (threadIdx.x == 0 && total) *total = run;
}

// With `fused`, sums[0, nc) are the raw chunk totals (not scanned): the
// workgroup of chunk c adds up those before c itself (nc <= kFusedChunks:
// at most 8 loads per thread), and chunk 0's workgroup writes the grand
// total. This saves the scan launch between the two passes.
constexpr int64_t kFusedChunks = 2048;
__device__ __forceinline__ int chunk_base(const int32_t* sums, int64_t nc, bool fused, int* lds,
                                          int32_t* total) {
  if (!fused) return sums[blockIdx.x];
  constexpr int kPer = static_cast<int>(kFusedChunks / kBlock);
  int v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int64_t j = threadIdx.x + static_cast<int64_t>(i) * kBlock;
    v[i] = j < nc ? sums[j] : 0;
  }
  int before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int64_t j = threadIdx.x + static_cast<int64_t>(i) * kBlock;
    all += v[i];
    before += j < static_cast<int64_t>(blockIdx.x) ? v[i] : 0;
  }
  int sum_before, sum_all;
  block_exclusive_scan<kBlock>(before, lds, &sum_before);
  block_exclusive_scan<kBlock>(all, lds, &sum_all);
  if (blockIdx.x == 0 && threadIdx.x == 0 && total) *total = sum_all;
  return sum_before;
}

__global__ void k_chunk_scan(int64_t n_max, const int32_t* n_dev, const int32_t* in, int32_t* out,
                             const int32_t* sums, bool fused, int64_t nc, int32_t* total) {
  __shared__ int lds[kWaves + 1];
  const int64_t n = live_count(n_max, n_dev);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
  if (base >= n) {  // uniform over the workgroup: the chunk is past the count
    if (fused && blockIdx.x == 0 && threadIdx.x == 0 && total) *total = 0;  // (n == 0)
    return;
  }
  int run = chunk_base(sums, nc, fused, lds, total);
  constexpr int R = kChunk / kBlock;
  int vals[R];
  chunk_values<R>(-1, in, base, n, vals);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (base + r * kBlock >= n) break;  // uniform: the rest of the chunk is past the count
    const int64_t p = base + r * kBlock + threadIdx.x;
    const int v = vals[r];
    int total;
    const int ex = block_exclusive_scan<kBlock>(v, lds, &total);
    if (p < n) out[p] = run + ex;
    run += total;
  }
}

__global__ void k_chunk_compact(int64_t n_max, const int32_t* n_dev, int32_t mode, const void* flags,
                                int32_t* out, const int32_t* sums, bool fused, int64_t nc, int32_t* total) {
  const int64_t n = live_count(n_max, n_dev);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
  __shared__ int wcnt[kWaves];
  __shared__ int lds[kWaves + 1];
  if (base >= n) {  // uniform over the workgroup: the chunk is past the count
    if (fused && blockIdx.x == 0 && threadIdx.x == 0 && total) *total = 0;  // (n == 0)
    return;
  }
  int run = chunk_base(sums, nc, fused, lds, total);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  constexpr int R = kChunk / kBlock;
  int fv[R];
  chunk_values<R>(mode, flags, base, n, fv);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (base + r * kBlock >= n) break;  // uniform: the rest of the chunk is past the count
    const int64_t p = base + r * kBlock + threadIdx.x;
    const int f = fv[r];
    const uint64_t m = __ballot(f);
    if (lane == 0) wcnt[wave] = __popcll(m);
    __syncthreads();
    int before = run;
    int total = 0;
    for (int w = 0; w < kWaves; ++w) {
      if (w < wave) before += wcnt[w];
      total += wcnt[w];
    }
    if (f) out[before + __popcll(m & lanemask_lt())] = static_cast<int32_t>(p);
    run += total;
    __syncthreads();
  }
}

// A radix pass's digit-by-tile counts are kept tile-major (t[tile * 256 + d])
// for up to kScanTilesMax tiles, and each scatter workgroup scans the table
// itself; larger tables are scanned digit-major by the chunked scan first.
constexpr int64_t kScanTilesMax = 256;

int64_t chunks_of(int64_t n) { return (n + kChunk - 1) / kChunk; }

// A fill kernel rather than hipMemsetAsync, so every node stays a kernel if a
// caller captures these launches in a graph.
__global__ void k_fill_i32(int64_t n, int32_t v, int32_t* out) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x)
    out[p] = v;
}

int scan_or_compact(int64_t n_max, const int32_t* n_dev, int32_t mode, const void* in, int32_t* out,
                    int32_t* total, int32_t* scratch, hipStream_t s, const char* what) {
  const int64_t nc = chunks_of(n_max);
  if (nc == 0) {
    if (total) hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(64), 0, s, int64_t(1), 0, total);
    return check_launch(what);
  }
  hipLaunchKernelGGL(k_chunk_sums, dim3(nc), dim3(kBlock), 0, s, n_max, n_dev, mode, in, scratch);
  // Up to kFusedChunks chunks the second pass adds up the chunk totals
  // itself; beyond, one workgroup scans them in between.
  const bool fused = nc <= kFusedChunks;
  if (!fused) hipLaunchKernelGGL(k_scan_single, dim3(1), dim3(kScanLanes), 0, s, nc, scratch, total);
  if (mode < 0)
    hipLaunchKernelGGL(k_chunk_scan, dim3(nc), dim3(kBlock), 0, s, n_max, n_dev,
                       static_cast<const int32_t*>(in), out, scratch, fused, nc, total);
  else
    hipLaunchKernelGGL(k_chunk_compact, dim3(nc), dim3(kBlock), 0, s, n_max, n_dev, mode, in, out,
                       scratch, fused, nc, total);
  return check_launch(what);
}

// ---------------------------------------------------------------------------
// Stable LSD radix sort.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t score_key(float f) {
  float k = (f != f) ? __builtin_huge_valf() : -f;
  if (k == 0.0f) k = 0.0f;  // -0 ties +0
  const uint32_t u = __float_as_uint(k);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Keys of R elements (the values being sorted, idx[r]; every idx[r] a valid
// index), with every load of a stage issued before any is used: the kind is
// uniform, so each case is straight-line code. Elements with ok[r] false get
// key 0 (their loads still go out, at a valid index).
template <int R>
__device__ __forceinline__ void sort_keys_of(const plx_sort_key& key, const uint32_t* idx, const bool* ok,
                                             uint32_t* k) {
  const int32_t* a = static_cast<const int32_t*>(key.a);
  switch (key.kind) {
    case PLX_KEY_SCORE: {
      float f[R];
#pragma unroll
      for (int r = 0; r < R; ++r) f[r] = static_cast<const float*>(key.a)[idx[r]];
#pragma unroll
      for (int r = 0; r < R; ++r) k[r] = ok[r] ? score_key(f[r]) : 0u;
      break;
    }
    case PLX_KEY_LEVEL_OF: {
      int32_t id[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        id[r] = a[idx[r]];
        if (key.bound > 0) id[r] = id[r] < 0 ? 0 : (id[r] >= key.bound ? key.bound - 1 : id[r]);
      }
      uint32_t lv[R];
#pragma unroll
      for (int r = 0; r < R; ++r) lv[r] = static_cast<uint32_t>(static_cast<const int32_t*>(key.b)[id[r]]);
#pragma unroll
      for (int r = 0; r < R; ++r) k[r] = ok[r] ? lv[r] : 0u;
      break;
    }
    case PLX_KEY_PAIR16: {
      uint32_t hi[R], lo[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        hi[r] = static_cast<uint32_t>(a[idx[r]]);
        lo[r] = static_cast<uint32_t>(static_cast<const int32_t*>(key.b)[idx[r]]);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) k[r] = ok[r] ? (hi[r] << 16) | (lo[r] & 0xFFFFu) : 0u;
      break;
    }
    case PLX_KEY_DEADMAX: {
      const uint32_t top = key.bits >= 32 ? 0xFFFFFFFFu : ((1u << key.bits) - 1u);
      uint32_t dv[R], av[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        dv[r] = static_cast<const uint8_t*>(key.b)[idx[r]];
        av[r] = static_cast<uint32_t>(a[idx[r]]);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) k[r] = ok[r] ? (dv[r] ? top : av[r]) : 0u;
      break;
    }
    default: {
      uint32_t av[R];
#pragma unroll
      for (int r = 0; r < R; ++r) av[r] = static_cast<uint32_t>(a[idx[r]]);
#pragma unroll
      for (int r = 0; r < R; ++r) k[r] = ok[r] ? av[r] : 0u;
      break;
    }
  }
}

// Per-tile digit counts at `shift`, digit-major (hist[d * ntiles + tile]).
// With GATHER the keys are computed from the values (sort_keys_of) and
// written to keys; vals_copy (optional) receives a copy of the values.
// The table's entry of (digit d, tile): tile-major when the scatter scans
// the table itself, else digit-major (the chunked scan's flat order).
__device__ __forceinline__ int64_t hist_at(bool tile_major, int d, int64_t tile, int64_t ntiles) {
  return tile_major ? tile * 256 + d : static_cast<int64_t>(d) * ntiles + tile;
}

// The radix kernels run kSortBlock threads per tile of kTile elements: R =
// 4 rounds of one element per thread. Each thread issues every load of its
// R elements before using any (one memory latency per tile, not one per
// round); the per-digit work (counters, the tile's digit offsets, the scan
// across the waves of a round) takes the first 256 threads.
constexpr int kSortBlock = 1024;
constexpr int kSortWaves = kSortBlock / 64;
static_assert(kTile % kSortBlock == 0, "a radix tile is whole rounds");

template <bool GATHER>
__global__ __launch_bounds__(kSortBlock) void k_radix_hist(int64_t n_max, const int32_t* n_dev, plx_sort_key key,
                                                           const uint32_t* vals, uint32_t* keys,
                                                           uint32_t* vals_copy, int shift, int64_t ntiles,
                                                           bool tile_major, int32_t* hist) {
  constexpr int R = kTile / kSortBlock;
  __shared__ int h[256];
  const int t = threadIdx.x;
  const int64_t n = live_count(n_max, n_dev);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  if (base >= n) {  // a tile past the count has no element (uniform over the workgroup)
    if (t < 256) hist[hist_at(tile_major, t, blockIdx.x, ntiles)] = 0;
    return;
  }
  if (t < 256) h[t] = 0;
  uint32_t k[R];
  if (GATHER) {
    uint32_t idx[R];
    bool ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      // (positions past the count read the last element: a valid index)
      const int64_t p = base + r * kSortBlock + t;
      ok[r] = p < n;
      idx[r] = vals[ok[r] ? p : n - 1];
    }
    sort_keys_of<R>(key, idx, ok, k);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t p = base + r * kSortBlock + t;
      if (ok[r]) {
        keys[p] = k[r];
        if (vals_copy) vals_copy[p] = idx[r];
      }
    }
  } else {
    uint32_t kv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t p = base + r * kSortBlock + t;
      kv[r] = keys[p < n ? p : n - 1];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) k[r] = base + r * kSortBlock + t < n ? kv[r] : 0u;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (base + r * kSortBlock + t < n) atomicAdd(&h[(k[r] >> shift) & 255u], 1);
  __syncthreads();
  if (t < 256) hist[hist_at(tile_major, t, blockIdx.x, ntiles)] = h[t];
}

__global__ __launch_bounds__(kSortBlock) void k_radix_scatter(int64_t n_max, const int32_t* n_dev,
                                                              const uint32_t* keys_in, const uint32_t* vals_in,
                                                              uint32_t* keys_out, uint32_t* vals_out, int shift,
                                                              int64_t ntiles, bool tile_major,
                                                              const int32_t* hist) {
  __shared__ int s_off[256];
  __shared__ int s_wcnt[kSortWaves][256];
  __shared__ int scan_lds[kSortWaves + 1];
  const int64_t n = live_count(n_max, n_dev);
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  if (base >= n) return;  // uniform over the workgroup
  // Every key and value of the thread's rounds is loaded first.
  constexpr int R = kTile / kSortBlock;
  uint32_t kr[R], vr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t p = base + r * kSortBlock + t;
    kr[r] = keys_in[p < n ? p : n - 1];  // (past the count: read but unused)
    vr[r] = vals_in[p < n ? p : n - 1];
  }
  if (tile_major) {
    // The raw digit-by-tile counts (tile-major, at most kScanTilesMax
    // tiles): thread t < 256 takes digit t. Its first output position is
    // the count of smaller digits over all tiles plus the count of digit t
    // in earlier tiles; every workgroup reads the whole table (one launch
    // fewer per pass than scanning it in its own kernel).
    // Four threads per digit (quarter q takes tiles q, q + 4, ...), each
    // issuing its loads in batches of 16: one memory round trip for up to
    // 64 tiles.
    constexpr int kBatch = 16;
    constexpr int kQuarters = kSortBlock / 256;
    __shared__ int part_total[kQuarters][256], part_before[kQuarters][256];
    const int dg = t & 255, q = t >> 8;
    int total = 0, before = 0;
    for (int64_t j0 = q; j0 < ntiles; j0 += kBatch * kQuarters) {
      int c[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) c[j] = hist[min(j0 + j * kQuarters, ntiles - 1) * 256 + dg];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int64_t tile = j0 + j * kQuarters;
        const int v = tile < ntiles ? c[j] : 0;
        total += v;
        before += tile < static_cast<int64_t>(blockIdx.x) ? v : 0;
      }
    }
    part_total[q][dg] = total;
    part_before[q][dg] = before;
    __syncthreads();
    total = 0;
    before = 0;
    if (t < 256) {
#pragma unroll
      for (int i = 0; i < kQuarters; ++i) {
        total += part_total[i][t];
        before += part_before[i][t];
      }
    }
    int all;
    const int ex = block_exclusive_scan<kSortBlock>(total, scan_lds, &all);
    if (t < 256) s_off[t] = ex + before;
  } else if (t < 256) {
    s_off[t] = hist[hist_at(tile_major, t, blockIdx.x, ntiles)];
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (base + r * kSortBlock >= n) break;  // uniform: the rest of the tile is past the count
    for (int i = t; i < kSortWaves * 256; i += kSortBlock) (&s_wcnt[0][0])[i] = 0;
    __syncthreads();
    const int64_t p = base + r * kSortBlock + t;
    const bool valid = p < n;
    const uint32_t key = kr[r];
    const uint32_t val = vr[r];
    const uint32_t d = (key >> shift) & 255u;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const bool on = (d >> bit) & 1u;
      const uint64_t b = __ballot(on);
      peers &= on ? b : ~b;
    }
    const int lrank = __popcll(peers & lanemask_lt());
    if (valid && lane == __ffsll(static_cast<long long>(peers)) - 1) s_wcnt[wave][d] = __popcll(peers);
    __syncthreads();
    if (t < 256) {
      int run = s_off[t];
      for (int w = 0; w < kSortWaves; ++w) {
        const int c = s_wcnt[w][t];
        s_wcnt[w][t] = run;
        run += c;
      }
      s_off[t] = run;
    }
    __syncthreads();
    if (valid) {
      const int pos = s_wcnt[wave][d] + lrank;
      keys_out[pos] = key;
      vals_out[pos] = val;
    }
    __syncthreads();
  }
}

// A sort of at most kSortSmall elements in one workgroup and one launch:
// each element's key tuple (every key masked to its bits) goes to LDS, and
// its rank is the number of elements before it in the order the LSD passes
// give (the last key most significant; equal tuples keep their positions).
constexpr int kSortSmall = 1024;
__global__ __launch_bounds__(kSortSmall) void k_sort_small(int64_t n_max, const int32_t* n_dev,
                                                           plx_sort_desc d) {
  __shared__ uint32_t kt[6][kSortSmall];
  const int t = threadIdx.x;
  const int n = static_cast<int>(live_count(n_max, n_dev));
  // Nothing to sort (uniform). Below, threads past the count compute their
  // keys at vals[0], a listed element, so every key load stays in bounds:
  // with no element, vals[0] is not one.
  if (n == 0) return;
  const bool ok = t < n;
  const uint32_t v = ok ? d.vals[t] : 0u;
  for (int q = 0; q < d.nkeys; ++q) {
    const plx_sort_key& key = d.keys[q];
    uint32_t k;
    const uint32_t idx[1] = {ok ? v : d.vals[0]};
    const bool okk[1] = {ok};
    sort_keys_of<1>(key, idx, okk, &k);
    const uint32_t mask = key.bits >= 32 ? 0xFFFFFFFFu : ((1u << key.bits) - 1u);
    kt[q][t] = k & mask;
  }
  __syncthreads();
  int rank = 0;
  if (ok) {
    for (int j = 0; j < n; ++j) {
      if (j == t) continue;
      int cmp = 0;  // -1: j before t, 1: t before j
      for (int q = d.nkeys - 1; q >= 0 && cmp == 0; --q) {
        const uint32_t a = kt[q][j], b = kt[q][t];
        cmp = a < b ? -1 : (a > b ? 1 : 0);
      }
      rank += (cmp < 0 || (cmp == 0 && j < t)) ? 1 : 0;
    }
  }
  __syncthreads();
  if (ok) d.vals[rank] = v;
}

int grid_for(int64_t n) {
  const int64_t g = (n + kBlock - 1) / kBlock;
  return static_cast<int>(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

// ---------------------------------------------------------------------------
// Site programs (the interpreter is in px_site.h).
// ---------------------------------------------------------------------------

// One step of a batched mean-of-writes update over a float32 column
// (phases.py:497-531: total of the per-sample changes in sample order, then
// old + total / batch).
__global__ void k_mean_of_writes(int64_t n, int32_t mode, int32_t batch, float* old, const float* next,
                                 float* total) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (mode == PLX_MOW_FIRST)
      total[i] = next[i] - old[i];
    else if (mode == PLX_MOW_ADD)
      total[i] = total[i] + (next[i] - old[i]);
    else
      old[i] = old[i] + total[i] / static_cast<float>(batch);
  }
}

__device__ __forceinline__ float gen_op(int32_t m, float a, float b) {
  switch (m) {
    case PLX_MONOID_PROD: return a * b;
    case PLX_MONOID_MAX: return fmax_nan(a, b);
    case PLX_MONOID_MIN: return fmin_nan(a, b);
    default: return a + b;
  }
}

__global__ void k_gen_fold(plx_gen_fold_desc d) {
  const uint32_t keyed = px::philox32(0, 1);  // the rng key of an unseeded step-0 site
  const int64_t B = d.batch > 1 ? d.batch : 1;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < d.nrows * B;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = t / B;
    const int32_t smp = static_cast<int32_t>(t - r * B);
    const int32_t u = d.row_unit[r];
    float s[8];
    for (int k = 0; k < 8; ++k) s[k] = d.identity[k];
    const int32_t* lg = d.ids_logical;
    const int32_t uu = lg ? lg[u] : u;
    for (int32_t j = d.row_ptr[r]; j < d.row_ptr[r + 1]; ++j) {
      const int64_t p = d.entry_pos ? d.entry_pos[j] : j;
      if (d.dead && d.dead[p]) continue;
      Site c;
      c.role[0] = c.role[1] = 0;
      if (d.backward) {
        c.role[2] = uu;
        c.role[3] = lg ? lg[d.to_id[p]] : d.to_id[p];
      } else {
        c.role[2] = lg ? lg[d.from_id[p]] : d.from_id[p];
        c.role[3] = uu;
      }
      const int32_t site = static_cast<int32_t>(p - d.base);
      c.role[4] = site;
      c.cid_value = d.slot ? d.slot[site] : site;
      c.seed = static_cast<uint64_t>(keyed) << 32;
      c.ids_logical = d.ids_logical;
      c.ids_physical = d.ids_physical;
      c.batch = static_cast<int32_t>(B);
      c.sample = smp;
      uint32_t out[PLX_MAX_SOUTS];
      for (int k = 0; k < PLX_MAX_SOUTS; ++k) out[k] = 0;
      site_run(d.prog, c, d.num_units, out);
      // (unrolled with a guard: constant indices keep out and s in registers)
#pragma unroll
      for (int k = 0; k < PLX_MAX_SOUTS; ++k)
        if (k < d.ncomp) s[k] = gen_op(d.monoid[k], s[k], __uint_as_float(out[k]));
    }
    const int64_t at = static_cast<int64_t>(u) * B + smp;
#pragma unroll
    for (int k = 0; k < PLX_MAX_SOUTS; ++k)
      if (k < d.ncomp) d.acc[k][at] = gen_op(d.monoid[k], d.acc[k][at], s[k]);
  }
}

__global__ void k_site_eval(plx_site_desc d) { site_eval_body<SiteInterp>(d); }

// ---------------------------------------------------------------------------
// Growth: validity, dedupe, selection, claim.
// ---------------------------------------------------------------------------

__device__ __forceinline__ bool live_pair(const plx_grow_filter_desc& d, int64_t nlive, int32_t b, int32_t s,
                                          int32_t t) {
  int64_t lo = 0, hi = nlive;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    const int32_t j = d.live_idx[mid];
    const int32_t jb = d.live_bucket[j], js = d.live_src[j], jd = d.live_dst[j];
    const bool less = jb < b || (jb == b && (js < s || (js == s && jd < t)));
    if (less)
      lo = mid + 1;
    else
      hi = mid;
  }
  if (lo >= nlive) return false;
  const int32_t j = d.live_idx[lo];
  return d.live_bucket[j] == b && d.live_src[j] == s && d.live_dst[j] == t;
}

__global__ void k_grow_filter(plx_grow_filter_desc d) {
  const int32_t nu = d.num_units;
  const int64_t nlive = live_count(d.nlive, d.nlive_dev);
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; s < d.n;
       s += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int32_t a = d.src[s], b = d.dst[s];
    bool ok = true;
    if (d.check_range) {
      if (!(a >= 0 && a < nu && b >= 0 && b < nu)) {
        ok = false;
        a = 0;
        b = 0;
      }
      d.src[s] = a;
      d.dst[s] = b;
    }
    a = a < 0 ? 0 : (a >= nu ? nu - 1 : a);
    b = b < 0 ? 0 : (b >= nu ? nu - 1 : b);
    if (d.proposer_dead) {
      const int64_t r = s / (d.per > 0 ? d.per : 1);
      const int64_t who = d.proposer_idx ? d.proposer_idx[r] : r;
      ok = ok && d.proposer_dead[who] == 0;
    }
    if (d.pruned) ok = ok && d.pruned[a] == 0 && d.pruned[b] == 0;
    const int32_t la = d.level[a], lb = d.level[b];
    const int32_t gap = lb - la;
    ok = ok && (gap < 0 ? -gap : gap) <= d.max_level_gap;
    if (!d.allow_self_loops) ok = ok && a != b;
    if (d.direction == 1) ok = ok && lb > la;
    if (d.direction == 2) ok = ok && lb >= la;
    int32_t bucket = 0;
    if (!d.pipeline) {
      bucket = la;
      ok = ok && la >= 0 && la < d.num_buckets;
      if (d.grid_sq > 0) ok = ok && static_cast<int64_t>(la) == s / d.grid_sq;
    }
    if (ok && nlive > 0) ok = !live_pair(d, nlive, bucket, a, b);
    if (!ok) d.score[s] = -__builtin_huge_valf();
  }
}

__global__ void k_mark_repeats(int64_t n_max, const int32_t* n_dev, const int32_t* order,
                               const int32_t* src, const int32_t* dst, float* score) {
  const int64_t n = live_count(n_max, n_dev);
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x + 1; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t i = order[p], h = order[p - 1];
    if (src[i] == src[h] && dst[i] == dst[h]) score[i] = -__builtin_huge_valf();
  }
}

__global__ void k_seg_first(int64_t n_max, const int32_t* n_dev, const int32_t* sorted,
                            const int32_t* src, const int32_t* level, int32_t* first) {
  const int64_t n = live_count(n_max, n_dev);
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t seg = level[src[sorted[p]]];
    if (p == 0 || level[src[sorted[p - 1]]] != seg) first[seg] = static_cast<int32_t>(p);
  }
}

__global__ void k_select(int64_t n_max, const int32_t* n_dev, const int32_t* sorted, const int32_t* src,
                         const int32_t* level, int32_t per_segment, int64_t k, const int32_t* first,
                         uint8_t* win) {
  const int64_t n = live_count(n_max, n_dev);
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t rank = p;
    if (per_segment) rank = p - first[level[src[sorted[p]]]];
    win[p] = rank < k;
  }
}

__device__ __forceinline__ int32_t level_of_winner(const plx_grow_claim_desc& d, int64_t q) {
  return d.level[d.src[d.winners[q]]];
}

__global__ void k_claim_growable(plx_grow_claim_desc d, int32_t* g) {
  const int64_t n = live_count(d.n_max, d.n_dev);
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < n;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (d.dropped_out) d.dropped_out[q] = 0;
    if (d.growable_in) {
      g[q] = d.growable_in[q] != 0;
      continue;
    }
    const float f = d.score[d.winners[q]];
    bool ok = (__float_as_uint(f) & 0x7F800000u) != 0x7F800000u;
    if (d.has_threshold) ok = ok && f >= d.threshold;
    g[q] = ok;
  }
}

__global__ void k_claim_cap(plx_grow_claim_desc d, const int32_t* g, const int32_t* scan, int32_t* g2) {
  const int64_t n = live_count(d.n_max, d.n_dev);
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < n;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x)
    g2[q] = g[q] && scan[q] < d.max_new_per_step;
}

// rank[q]: q's rank among its level's growable winners; spill[q] (PIPELINE):
// growable and past its level's own dead slots.
__global__ void k_claim_rank(plx_grow_claim_desc d, const int32_t* g, const int32_t* scan, int32_t* rank,
                             int32_t* spill) {
  const int64_t n = live_count(d.n_max, d.n_dev);
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < n;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t lvl = level_of_winner(d, q);
    int64_t lo = 0, hi = q;  // first position of this level's run
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (level_of_winner(d, mid) < lvl)
        lo = mid + 1;
      else
        hi = mid;
    }
    const int32_t rk = scan[q] - scan[lo];
    rank[q] = rk;
    if (d.pipeline) {
      const int32_t own = d.own_count[lvl < d.num_levels ? lvl : d.num_levels - 1];
      spill[q] = g[q] && rk >= own;
    } else {
      spill[q] = 0;
    }
  }
}

__global__ void k_claim_write(plx_grow_claim_desc d, const int32_t* g, const int32_t* rank,
                              const int32_t* spill, const int32_t* spill_rank) {
  const int64_t n = live_count(d.n_max, d.n_dev);
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < n;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (!g[q]) continue;
    const int32_t w = d.winners[q];
    const int32_t a = d.src[w], b = d.dst[w];
    const int32_t lvl = d.level[a];
    int64_t slot = -1;
    if (!d.pipeline) {
      const int32_t start = d.free_info[2 * lvl], len = d.free_info[2 * lvl + 1];
      if (rank[q] < len) slot = d.free_slots[start + rank[q]];
    } else if (!spill[q]) {
      const int32_t l = lvl < d.num_levels ? lvl : d.num_levels - 1;
      slot = d.own_slots[d.own_start[l] + rank[q]];
    } else {
      const int64_t t = (d.tail_dev ? static_cast<int64_t>(*d.tail_dev) : d.tail_start) + spill_rank[q];
      if (t < d.capacity) {
        slot = t;
        atomicAdd(&d.flags[3], 1);
      }
    }
    if (slot < 0) {
      atomicOr(&d.flags[1], 1);
      if (d.dropped_out) d.dropped_out[q] = 1;
      continue;
    }
    atomicAdd(&d.flags[0], 1);
    if (d.level[b] <= lvl) atomicOr(&d.flags[2], 1);
    if (d.claimed_out) {
      const int i = atomicAdd(d.claimed_n, 1);
      if (i < d.claimed_cap) d.claimed_out[i] = static_cast<int32_t>(slot);
    }
    d.from_id[slot] = a;
    d.to_id[slot] = b;
    d.dead[slot] = 0;
    for (int c = 0; c < d.ncols; ++c) {
      const plx_grow_col& col = d.cols[c];
      const uint32_t v = col.init_slot >= 0 ? d.init_out[col.init_slot][q] : col.default_bits;
      if (col.bytes == 1)
        static_cast<uint8_t*>(col.ptr)[slot] = v != 0u;
      else
        static_cast<uint32_t*>(col.ptr)[slot] = v;
    }
  }
}

// The new tail start after a PIPELINE claim: the old one plus the tail slots
// it used.
__global__ void k_claim_tail(const int32_t* tail_dev, int32_t* flags) {
  if (threadIdx.x == 0) flags[4] = *tail_dev + flags[3];
}

__global__ void k_gather_level(int64_t n_max, const int32_t* n_dev, const int32_t* idx, const int32_t* ids,
                               const int32_t* level, int32_t bound, int32_t* out) {
  const int64_t n = live_count(n_max, n_dev);
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int32_t o = ids[idx[p]];
    o = o < 0 ? 0 : (o > bound - 1 ? bound - 1 : o);
    out[p] = level[o];
  }
}

__global__ void k_occurrence(int64_t n, const int32_t* sorted, const int32_t* from_id,
                             const int32_t* to_id, int32_t* occ) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t i = sorted[p];
    const int32_t s = from_id[i], t = to_id[i];
    int64_t lo = 0, hi = p;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      const int32_t j = sorted[mid];
      const bool less = from_id[j] < s || (from_id[j] == s && to_id[j] < t);
      if (less)
        lo = mid + 1;
      else
        hi = mid;
    }
    occ[i] = static_cast<int32_t>(p - lo);
  }
}

__global__ void k_gather_i32(int64_t n_max, const int32_t* n_dev, const int32_t* idx, const int32_t* a,
                             int32_t* out) {
  const int64_t n = live_count(n_max, n_dev);
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x)
    out[p] = a[idx[p]];
}

__global__ void k_level_count(int64_t n_max, const int32_t* n_dev, const int32_t* keys, int32_t nl,
                              int32_t* count) {
  const int64_t n = live_count(n_max, n_dev);
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t k = keys[p];
    if (k >= 0 && k < nl) atomicAdd(&count[k], 1);
  }
}

__global__ void k_copy_i32(int64_t n, const int32_t* in, int32_t* out) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x)
    out[p] = in[p];
}

__global__ void k_bucket_free(int32_t nb, const int64_t* off, const int32_t* free_slots,
                              const int32_t* ntotal, int32_t* info) {
  const int32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nb) return;
  const int64_t total = *ntotal;
  auto lower = [&](int64_t v) {
    int64_t lo = 0, hi = total;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (free_slots[mid] < v)
        lo = mid + 1;
      else
        hi = mid;
    }
    return lo;
  };
  const int64_t s = lower(off[b]), e = lower(off[b + 1]);
  info[2 * b] = static_cast<int32_t>(s);
  info[2 * b + 1] = static_cast<int32_t>(e - s);
}

__global__ void k_mask_importance(int32_t n, const float* imp, const int32_t* level, const uint8_t* pruned,
                                  int32_t mode, int32_t b, int32_t gap, int32_t direction, float* out) {
  const int32_t u = blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= n) return;
  const int32_t l = level[u];
  bool ok = true;
  if (mode == 0) {
    ok = l == b;
  } else if (mode == 1) {
    const int32_t dl = l - b;
    ok = (dl < 0 ? -dl : dl) <= gap;
    if (direction == 1) ok = ok && l > b;
    if (direction == 2) ok = ok && l >= b;
  }
  if (pruned && pruned[u]) ok = false;
  out[u] = ok ? imp[u] : -__builtin_huge_valf();
}

// ---------------------------------------------------------------------------
// Unit lifecycle.
// ---------------------------------------------------------------------------

struct UnitCols {
  plx_unit_col c[PLX_MAX_UNIT_COLS];
  int32_t n;
};

__device__ __forceinline__ void unit_store(const plx_unit_col& col, int64_t u, uint32_t v) {
  if (col.bytes == 1)
    static_cast<uint8_t*>(col.ptr)[u] = v != 0u;
  else
    static_cast<uint32_t*>(col.ptr)[u] = v;
}

struct UnitOuts {
  const uint32_t* o[PLX_MAX_UNIT_COLS];
};

__global__ void k_unit_write(int64_t n_max, const int32_t* n_dev, const int32_t* idx, const uint8_t* skip,
                             UnitCols cols, UnitOuts outs) {
  const int64_t n = live_count(n_max, n_dev);
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; r < n;
       r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t u = idx ? idx[r] : r;
    if (skip && skip[u]) continue;
    for (int k = 0; k < cols.n; ++k) unit_store(cols.c[k], u, outs.o[k][r]);
  }
}

__global__ void k_unit_prune(int64_t n, const uint32_t* selected, uint8_t* pruned, const uint8_t* exempt,
                             UnitCols cols, uint8_t* doomed, int32_t* count) {
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < n;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const bool d = selected[u] != 0u && !pruned[u] && !(exempt && exempt[u]);
    doomed[u] = d;
    if (!d) continue;
    for (int k = 0; k < cols.n; ++k) unit_store(cols.c[k], u, cols.c[k].default_bits);
    pruned[u] = 1;
    if (count) atomicAdd(count, 1);
  }
}

// start[u] = the number of keys below u (lower bound of u in the ascending
// keys), u in [0, nlevels]: a CSR's offsets from its sorted row ids.
__global__ void k_sorted_starts(int64_t n_max, const int32_t* n_dev, const int32_t* keys, int32_t nlevels,
                                int32_t* start) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (u > nlevels) return;
  const int64_t n = live_count(n_max, n_dev);
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (keys[mid] < u)
      lo = mid + 1;
    else
      hi = mid;
  }
  start[u] = static_cast<int32_t>(lo);
}

__global__ void k_merge_kills(int64_t n, const uint8_t* sink, uint8_t* dead, float* stamp, float stamp_value) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (sink[p] && !dead[p]) {
      dead[p] = 1;
      if (stamp) stamp[p] = stamp_value;
    }
  }
}

__global__ void k_kill_incident(int64_t n, const int32_t* from_id, const int32_t* to_id, uint8_t* dead,
                                const uint8_t* doomed, const int32_t* id_map, int32_t* count, float* stamp,
                                float stamp_value) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (dead[p]) continue;  // already a tombstone: its ids are not read
    int32_t a = from_id[p], b = to_id[p];
    if (id_map) {
      a = id_map[a];
      b = id_map[b];
    }
    if (doomed[a] || doomed[b]) {
      dead[p] = 1;
      if (stamp) stamp[p] = stamp_value;
      if (count) atomicAdd(count, 1);
    }
  }
}

__global__ void k_unit_place(int64_t n_max, const int32_t* parents, const int32_t* nparents, const int32_t* free_ids,
                             const int32_t* nfree, const int32_t* offset, int32_t* level, uint8_t* pruned,
                             int32_t max_level, UnitCols cols, int32_t* child, int32_t* parent, int32_t* flags) {
  const int64_t np = *nparents, nf = *nfree;
  const int64_t placed = np < nf ? np : nf;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    flags[0] = static_cast<int32_t>(placed);
    flags[1] = np > nf;
  }
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; r < placed && r < n_max;
       r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t p = parents[r], c = free_ids[r];
    for (int k = 0; k < cols.n; ++k) unit_store(cols.c[k], c, cols.c[k].default_bits);
    int32_t l = level[p] + offset[p];
    l = l < 1 ? 1 : (l > max_level ? max_level : l);
    level[c] = l;
    pruned[c] = 0;
    child[r] = c;
    parent[r] = p;
  }
}

// ---------------------------------------------------------------------------
// Resort.
// ---------------------------------------------------------------------------

__global__ void k_relax_edges(int64_t n, const int32_t* from_id, const int32_t* to_id, const uint8_t* dead,
                              const int32_t* level_in, int32_t* level_out) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (dead[p]) continue;
    atomicMax(&level_out[to_id[p]], level_in[from_id[p]] + 1);
  }
}

__global__ void k_pin_compare(int64_t n, const int32_t* level_in, int32_t* level_out, const uint8_t* is_input,
                              int32_t* changed) {
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < n;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (is_input && is_input[u]) level_out[u] = 0;
    if (level_out[u] != level_in[u]) atomicOr(changed, 1);
  }
}

__global__ void k_resort_keys(int64_t n, const int32_t* from_id, const uint8_t* dead, const int32_t* level,
                              int32_t pipeline, int32_t sentinel, int32_t* key) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x)
    key[p] = dead[p] ? sentinel : (pipeline ? 0 : level[from_id[p]]);
}

__global__ void k_gather_col(int64_t n_max, const int32_t* n_dev, const int32_t* idx, const void* src, void* dst,
                             int32_t bytes) {
  const int64_t n = live_count(n_max, n_dev);
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (bytes == 1)
      static_cast<uint8_t*>(dst)[p] = static_cast<const uint8_t*>(src)[idx[p]];
    else
      static_cast<uint32_t*>(dst)[p] = static_cast<const uint32_t*>(src)[idx[p]];
  }
}

bool unit_cols_ok(int32_t ncols, const plx_unit_col* cols) {
  if (ncols < 0 || ncols > PLX_MAX_UNIT_COLS || (ncols > 0 && !cols)) return false;
  for (int k = 0; k < ncols; ++k)
    if (!cols[k].ptr || (cols[k].bytes != 1 && cols[k].bytes != 4)) return false;
  return true;
}

UnitCols pack_cols(int32_t ncols, const plx_unit_col* cols) {
  UnitCols u{};
  u.n = ncols;
  for (int k = 0; k < ncols; ++k) u.c[k] = cols[k];
  return u;
}

// Descriptors travel by value as kernel arguments (4 KB at most).
static_assert(sizeof(plx_site_desc) <= 3584, "plx_site_desc must fit the kernel-argument segment");

bool prog_ok(const plx_site_prog& p) {
  if (p.ninstr < 0 || p.ninstr > PLX_MAX_SINSTR || p.nout < 0 || p.nout > PLX_MAX_SOUTS) return false;
  for (int k = 0; k < p.ninstr; ++k) {
    const int op = p.code[4 * k], d = p.code[4 * k + 1], a = p.code[4 * k + 2], b = p.code[4 * k + 3];
    if (op == S_OUT) {
      if (d < 0 || d >= p.nout || a < 0 || a >= 32) return false;
      continue;
    }
    if (d < 0 || d >= 32) return false;
    if (op == S_CONST && (a < 0 || a >= PLX_MAX_SCONST)) return false;
    if (op == S_IDX && (a < 0 || a >= 5)) return false;
    if (op == S_LDU && (a < 0 || a >= PLX_MAX_SFIELDS || !p.ufields[a] || b < 0 || b >= 32)) return false;
    if (op == S_LDC && (a < 0 || a >= PLX_MAX_SFIELDS || !p.cfields[a])) return false;
    if (op == S_SEL && (b < 0 || b + 1 >= 32)) return false;
  }
  return true;
}

// ---------------------------------------------------------------------------
// Compiled site programs: a program's own kernel, generated as source (the
// shared site_eval_body with a runner that calls site_step once per
// instruction, operands as literals) and compiled with hipRTC for the
// current device, with the library's floating-point flags. One compile per
// (device, program code, launch shape); the modules stay loaded for the
// process.
// ---------------------------------------------------------------------------
struct CompiledSite {
  hipModule_t mod = nullptr;
  hipFunction_t fn = nullptr;
  int dev = -1;
  int32_t monoid = -1;  // < 0: plx_site_eval's kernel; else the forward + prune kernel for this monoid
  int32_t ninstr = 0, nout = 0;
  std::vector<int32_t> code;
  std::vector<int32_t> shape;  // site_shape of the descriptors it runs
};

// What a compiled kernel fixes besides the code: the site kind, whether the
// unit columns are batched, which optional id arrays are passed, and every
// field's width (and id-column flag). A descriptor runs on the kernel only
// with the same values.
std::vector<int32_t> site_shape(const plx_site_desc& d) {
  std::vector<int32_t> v = {d.kind,
                            d.batch > 1,
                            d.from_id != nullptr,
                            d.to_id != nullptr,
                            d.site_ids != nullptr,
                            d.ids_logical != nullptr,
                            d.ids_physical != nullptr};
  v.insert(v.end(), d.prog.ubytes, d.prog.ubytes + PLX_MAX_SFIELDS);
  v.insert(v.end(), d.prog.cbytes, d.prog.cbytes + PLX_MAX_SFIELDS);
  return v;
}

std::mutex g_site_mu;
std::map<std::string, CompiledSite*> g_site_cache;

// The generated program after `header`: its launch shape (SiteShape) and
// instructions (SiteGen), in an anonymous namespace.
std::string site_gen_source(const plx_site_desc& d, const char* header) {
  const plx_site_prog& p = d.prog;
  const std::vector<int32_t> sh = site_shape(d);
  auto b = [](bool v) { return std::string(v ? "true" : "false"); };
  auto widths = [](const int32_t* w) {
    std::string t = "switch (a) {";
    for (int f = 0; f < PLX_MAX_SFIELDS; ++f) t += " case " + std::to_string(f) + ": return " + std::to_string(w[f]) + ";";
    return t + " default: return 4; }";
  };
  std::string s =
      "// generated by plx_site_compile: one site program, its instructions as site_step calls\n"
      "using __hip_internal::int8_t;\nusing __hip_internal::uint8_t;\nusing __hip_internal::int16_t;\n"
      "using __hip_internal::uint16_t;\nusing __hip_internal::int32_t;\nusing __hip_internal::uint32_t;\n"
      "using __hip_internal::int64_t;\nusing __hip_internal::uint64_t;\n"
      "#ifndef INT32_MIN\n#define INT32_MIN (-2147483647 - 1)\n#endif\n"
      "#ifndef INT32_MAX\n#define INT32_MAX 2147483647\n#endif\n"
      "#ifndef UINT32_MAX\n#define UINT32_MAX 4294967295u\n#endif\n"
      "#include \"" + std::string(header) + "\"\n"
      "namespace {\n"
      "struct SiteShape {\n"
      "  static constexpr bool kSelects = true;\n"
      "  __device__ __forceinline__ static int kind(const plx_site_desc&) { return " + std::to_string(sh[0]) + "; }\n"
      "  __device__ __forceinline__ static int32_t batch(const plx_site_desc& d) { return " +
      std::string(sh[1] ? "d.batch" : "1") + "; }\n"
      "  __device__ __forceinline__ static bool from(const plx_site_desc&) { return " + b(sh[2]) + "; }\n"
      "  __device__ __forceinline__ static bool to(const plx_site_desc&) { return " + b(sh[3]) + "; }\n"
      "  __device__ __forceinline__ static bool site_ids(const plx_site_desc&) { return " + b(sh[4]) + "; }\n"
      "  __device__ __forceinline__ static bool logical(const Site&) { return " + b(sh[5]) + "; }\n"
      "  __device__ __forceinline__ static bool physical(const Site&) { return " + b(sh[6]) + "; }\n"
      "  __device__ __forceinline__ static bool batched(const Site&) { return " + b(sh[1]) + "; }\n"
      "  __device__ __forceinline__ static int32_t ubytes(const plx_site_prog&, int a) { " + widths(p.ubytes) + " }\n"
      "  __device__ __forceinline__ static int32_t cbytes(const plx_site_prog&, int a) { " + widths(p.cbytes) + " }\n"
      "};\n"
      "struct SiteGen {\n"
      "  using Shape = SiteShape;\n"
      "  static constexpr int kSites = 4;\n"
      "  __device__ __forceinline__ static void run(const plx_site_prog& p, const Site& c, int32_t nu,\n"
      "                                             uint32_t (&o)[PLX_MAX_SOUTS]) {\n"
      "    SiteRegs r;\n";
  for (int k = 0; k < p.ninstr; ++k) {
    s += "    site_step<SiteShape>(" + std::to_string(p.code[4 * k]) + ", " + std::to_string(p.code[4 * k + 1]) + ", " +
         std::to_string(p.code[4 * k + 2]) + ", " + std::to_string(p.code[4 * k + 3]) + ", r, p, c, nu, o);\n";
  }
  s += "  }\n};\n}  // namespace\n";
  return s;
}

// plx_site_eval's kernel for the program of d.
std::string site_source(const plx_site_desc& d) {
  return site_gen_source(d, "px_site.h") +
         "extern \"C\" __global__ void plx_site_kernel(plx_site_desc d) { site_eval_body<SiteGen>(d); }\n";
}

// The forward sweep with the PruneConn program of d compiled in
// (px_forward.h's forward_body), for monoid m.
std::string forward_prune_source(const plx_site_desc& d, int32_t m) {
  return site_gen_source(d, "px_forward.h") +
         "extern \"C\" __global__ __launch_bounds__(kFwdBlock) void plx_fwd_prune_kernel(plx_forward_desc d) {\n"
         "  forward_body<" + std::to_string(m) + ", true, SiteGen>(d);\n}\n";
}

int site_rtc_compile(const std::string& src, const char* csrc_dir, const std::string& arch, std::vector<char>* code) {
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "plx_site.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    return fail(PLX_ERR_HIP, "plx_site_compile: hiprtcCreateProgram failed");
  const std::string inc = std::string("-I") + csrc_dir;
  const std::string off = "--offload-arch=" + arch;
  const char* opts[] = {off.c_str(), "-O3", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", inc.c_str()};
  const hiprtcResult rc = hiprtcCompileProgram(prog, static_cast<int>(sizeof(opts) / sizeof(opts[0])), opts);
  if (rc != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    plx_detail::g_last_error = "plx_site_compile: " + std::string(hiprtcGetErrorString(rc)) + ": " + log.substr(0, 4000);
    return PLX_ERR_HIP;
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  code->assign(n, 0);
  hiprtcGetCode(prog, code->data());
  hiprtcDestroyProgram(&prog);
  return PLX_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI.
// ---------------------------------------------------------------------------

int64_t plx_scratch_ints(int64_t n) {
  const int64_t tiles = (n + kTile - 1) / kTile;
  const int64_t h = 256 * tiles;
  return h + chunks_of(h) + chunks_of(n) + 64;
}

// The checks of plx_site_eval for n > 0.
static int site_desc_check(const plx_site_desc* d) {
  if (!prog_ok(d->prog)) return fail(PLX_ERR_INVALID, "plx_site_eval: bad program");
  if (d->num_units < 1) return fail(PLX_ERR_INVALID, "plx_site_eval: num_units must be positive");
  if (d->kind < PLX_SITES_UNIT || d->kind > PLX_SITES_EDGE)
    return fail(PLX_ERR_INVALID, "plx_site_eval: unknown site kind");
  if (d->batch > 1 && (d->sample < 0 || d->sample >= d->batch))
    return fail(PLX_ERR_INVALID, "plx_site_eval: sample outside the batch");
  if (d->batch > 1 && d->kind == PLX_SITES_UNIT &&
      (d->site_ids ? d->n % d->batch != 0 : d->n != static_cast<int64_t>(d->num_units) * d->batch))
    return fail(PLX_ERR_INVALID,
                "plx_site_eval: batched unit sites are num_units * batch (site_ids: a multiple of batch)");
  if ((d->kind == PLX_SITES_CONN && (!d->list_a || !d->from_id || !d->to_id || !d->occ)) ||
      ((d->kind == PLX_SITES_GRID || d->kind == PLX_SITES_PAIRS) && (!d->list_a || !d->list_b)))
    return fail(PLX_ERR_INVALID, "plx_site_eval: site lists missing");
  if (!d->or_into)
    for (int k = 0; k < d->prog.nout; ++k)
      if (!d->outs[k]) return fail(PLX_ERR_INVALID, "plx_site_eval: null output");
  return PLX_OK;
}

int plx_site_eval(const plx_site_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_site_eval: null descriptor");
  if (d->n < 0) return fail(PLX_ERR_INVALID, "plx_site_eval: negative n");
  if (d->n == 0) return PLX_OK;
  const int rc = site_desc_check(d);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_site_eval, dim3(grid_for(d->n)), dim3(kBlock), 0, s, *d);
  return check_launch("plx_site_eval");
}



// plx_site_compile and plx_forward_prune_compile: the program of d compiled
// as plx_site_eval's kernel (monoid < 0) or inside the forward sweep for
// monoid m, loaded on the current device, once per (device, target, kernel,
// program code, launch shape) for the process.
static int compile_kernel(const plx_site_desc* d, int32_t monoid, const char* csrc_dir, const char* arch,
                          void** handle, const char* who) {
  const std::string w(who);
  if (!d || !csrc_dir) return fail(PLX_ERR_INVALID, (w + ": null argument").c_str());
  const plx_site_prog* p = &d->prog;
  if (d->kind < PLX_SITES_UNIT || d->kind > PLX_SITES_EDGE) return fail(PLX_ERR_INVALID, (w + ": bad site kind").c_str());
  if (p->ninstr < 0 || p->ninstr > PLX_MAX_SINSTR || p->nout < 0 || p->nout > PLX_MAX_SOUTS)
    return fail(PLX_ERR_INVALID, (w + ": bad program").c_str());
  std::string target = arch ? arch : "";
  int dev = -1;
  if (handle) {
    if (hipGetDevice(&dev) != hipSuccess) return fail(PLX_ERR_HIP, (w + ": no current device").c_str());
    if (target.empty()) {
      static std::mutex arch_mu;
      static std::map<int, std::string> arch_of;  // (device properties are slow to query)
      std::lock_guard<std::mutex> lock(arch_mu);
      auto it = arch_of.find(dev);
      if (it == arch_of.end()) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
          return fail(PLX_ERR_HIP, (w + ": device properties unavailable").c_str());
        it = arch_of.emplace(dev, std::string(prop.gcnArchName)).first;
      }
      target = it->second;
    }
  }
  if (target.empty()) return fail(PLX_ERR_INVALID, (w + ": no target architecture").c_str());
  std::string key = std::to_string(dev) + "|" + target + "|" + std::to_string(monoid) + "|" +
                    std::to_string(p->ninstr) + "|" + std::to_string(p->nout) + "|";
  key.append(reinterpret_cast<const char*>(p->code), sizeof(int32_t) * 4 * static_cast<size_t>(p->ninstr));
  const std::vector<int32_t> shape = site_shape(*d);
  key.append(reinterpret_cast<const char*>(shape.data()), sizeof(int32_t) * shape.size());
  std::lock_guard<std::mutex> lock(g_site_mu);
  if (handle) {
    const auto it = g_site_cache.find(key);
    if (it != g_site_cache.end()) {
      *handle = it->second;
      return PLX_OK;
    }
  }
  std::vector<char> code;
  const int rc = site_rtc_compile(monoid < 0 ? site_source(*d) : forward_prune_source(*d, monoid), csrc_dir, target,
                                  &code);
  if (rc || !handle) return rc;
  auto* cs = new CompiledSite;
  const char* name = monoid < 0 ? "plx_site_kernel" : "plx_fwd_prune_kernel";
  if (hipModuleLoadData(&cs->mod, code.data()) != hipSuccess ||
      hipModuleGetFunction(&cs->fn, cs->mod, name) != hipSuccess) {
    delete cs;
    (void)hipGetLastError();
    return fail(PLX_ERR_HIP, (w + ": loading the compiled program failed").c_str());
  }
  cs->dev = dev;
  cs->monoid = monoid;
  cs->ninstr = p->ninstr;
  cs->nout = p->nout;
  cs->code.assign(p->code, p->code + 4 * p->ninstr);
  cs->shape = shape;
  g_site_cache[key] = cs;
  *handle = cs;
  return PLX_OK;
}

int plx_site_compile(const plx_site_desc* d, const char* csrc_dir, const char* arch, void** handle) {
  return compile_kernel(d, -1, csrc_dir, arch, handle, "plx_site_compile");
}

int plx_forward_prune_compile(const plx_site_desc* d, int32_t monoid, const char* csrc_dir, const char* arch,
                              void** handle) {
  if (monoid < PLX_MONOID_SUM || monoid > PLX_MONOID_MIN)
    return fail(PLX_ERR_UNSUPPORTED, "plx_forward_prune_compile: unknown monoid");
  if (d && (d->kind != PLX_SITES_EDGE || d->batch > 1 || d->prog.nout < 1))
    return fail(PLX_ERR_INVALID, "plx_forward_prune_compile: the predicate is an unbatched EDGE site program "
                                 "with an output");
  return compile_kernel(d, monoid, csrc_dir, arch, handle, "plx_forward_prune_compile");
}

int plx_forward_bucket_compiled(void* handle, const plx_forward_desc* d, void* stream) {
  if (!handle || !d) return fail(PLX_ERR_INVALID, "plx_forward_bucket_compiled: null argument");
  const auto* cs = static_cast<const CompiledSite*>(handle);
  if (cs->monoid < 0) return fail(PLX_ERR_INVALID, "plx_forward_bucket_compiled: not a forward + prune kernel");
  if (d->monoid != cs->monoid)
    return fail(PLX_ERR_INVALID, "plx_forward_bucket_compiled: the descriptor's monoid is not the compiled one");
  if (!d->prune_prog) return fail(PLX_ERR_INVALID, "plx_forward_bucket_compiled: prune_prog is required");
  // (the kernel reads the id arrays the compiled shape names, unconditionally)
  if ((d->ids_logical != nullptr) != (cs->shape[5] != 0) || (d->ids_physical != nullptr) != (cs->shape[6] != 0))
    return fail(PLX_ERR_INVALID,
                "plx_forward_bucket_compiled: ids_logical / ids_physical are not set as in the compiled shape");
  unsigned grid = 0, block = 0;
  const int rc = plx_detail::forward_launch_shape(d, "plx_forward_bucket_compiled", &grid, &block);
  if (rc || grid == 0) return rc;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != cs->dev)
    return fail(PLX_ERR_INVALID, "plx_forward_bucket_compiled: the kernel was compiled for another device");
  void* args[] = {const_cast<plx_forward_desc*>(d)};
  if (hipModuleLaunchKernel(cs->fn, grid, 1, 1, block, 1, 1, 0, static_cast<hipStream_t>(stream), args, nullptr) !=
      hipSuccess)
    return fail(PLX_ERR_HIP, "plx_forward_bucket_compiled: launch failed");
  return check_launch("plx_forward_bucket_compiled");
}

int plx_site_eval_compiled(void* handle, const plx_site_desc* d, void* stream) {
  if (!handle || !d) return fail(PLX_ERR_INVALID, "plx_site_eval_compiled: null argument");
  if (static_cast<const CompiledSite*>(handle)->monoid >= 0)
    return fail(PLX_ERR_INVALID, "plx_site_eval_compiled: a forward + prune kernel, not a site kernel");
  if (d->n < 0) return fail(PLX_ERR_INVALID, "plx_site_eval: negative n");
  if (d->n == 0) return PLX_OK;
  const int rc = site_desc_check(d);
  if (rc) return rc;
  const auto* cs = static_cast<const CompiledSite*>(handle);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != cs->dev)
    return fail(PLX_ERR_INVALID, "plx_site_eval_compiled: the program was compiled for another device");
  if (cs->ninstr != d->prog.ninstr || cs->nout != d->prog.nout ||
      std::memcmp(cs->code.data(), d->prog.code, sizeof(int32_t) * 4 * static_cast<size_t>(cs->ninstr)) != 0)
    return fail(PLX_ERR_INVALID, "plx_site_eval_compiled: the descriptor's program is not the compiled one");
  if (site_shape(*d) != cs->shape)
    return fail(PLX_ERR_INVALID,
                "plx_site_eval_compiled: the descriptor's site kind, batch, id arrays or field widths are not the "
                "compiled ones");
  void* args[] = {const_cast<plx_site_desc*>(d)};
  // (four sites per lane per pass: SiteGen::kSites)
  if (hipModuleLaunchKernel(cs->fn, grid_for((d->n + 3) / 4), 1, 1, kBlock, 1, 1, 0,
                            static_cast<hipStream_t>(stream), args, nullptr) != hipSuccess)
    return fail(PLX_ERR_HIP, "plx_site_eval_compiled: launch failed");
  return check_launch("plx_site_eval_compiled");
}

int plx_mean_of_writes(int64_t n, int32_t mode, int32_t batch, float* old, const float* next, float* total,
                       void* stream) {
  if (n < 0 || mode < PLX_MOW_FIRST || mode > PLX_MOW_APPLY || batch < 1)
    return fail(PLX_ERR_INVALID, "plx_mean_of_writes: bad n, mode or batch");
  if (n == 0) return PLX_OK;
  if (!old || !total || (mode != PLX_MOW_APPLY && !next))
    return fail(PLX_ERR_INVALID, "plx_mean_of_writes: null column");
  hipLaunchKernelGGL(k_mean_of_writes, dim3(grid_for(n)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), n,
                     mode, batch, old, next, total);
  return check_launch("plx_mean_of_writes");
}

int plx_compact(int64_t n, const int32_t* n_dev, int32_t mode, const void* flags, int32_t* out,
                int32_t* count, int32_t* scratch, void* stream) {
  if (n < 0 || mode < 0 || mode > PLX_FLAG_I32) return fail(PLX_ERR_INVALID, "plx_compact: bad n or mode");
  if ((n > 0 && (!flags || !out || !scratch)) || !count) return fail(PLX_ERR_INVALID, "plx_compact: null pointer");
  return scan_or_compact(n, n_dev, mode, flags, out, count, scratch, static_cast<hipStream_t>(stream),
                         "plx_compact");
}

int plx_scan_i32(int64_t n, const int32_t* n_dev, const int32_t* in, int32_t* out, int32_t* total,
                 int32_t* scratch, void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_scan_i32: negative n");
  if (n > 0 && (!in || !out || !scratch)) return fail(PLX_ERR_INVALID, "plx_scan_i32: null pointer");
  return scan_or_compact(n, n_dev, -1, in, out, total, scratch, static_cast<hipStream_t>(stream),
                         "plx_scan_i32");
}

int plx_sort(const plx_sort_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_sort: null descriptor");
  if (d->n_max < 0 || d->nkeys < 0 || d->nkeys > 6) return fail(PLX_ERR_INVALID, "plx_sort: bad sizes");
  if (d->n_max == 0) return PLX_OK;
  if (!d->vals || !d->keys_buf || !d->keys_alt || !d->vals_alt || !d->hist)
    return fail(PLX_ERR_INVALID, "plx_sort: null buffer");
  if (d->n_max > (int64_t(1) << 31) - 1) return fail(PLX_ERR_UNSUPPORTED, "plx_sort: more than 2^31 - 1 elements");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (d->n_max <= kSortSmall) {
    for (int k = 0; k < d->nkeys; ++k) {
      const plx_sort_key& key = d->keys[k];
      if (key.bits < 1 || key.bits > 32 || !key.a) return fail(PLX_ERR_INVALID, "plx_sort: bad key");
      if ((key.kind == PLX_KEY_LEVEL_OF || key.kind == PLX_KEY_PAIR16 || key.kind == PLX_KEY_DEADMAX) && !key.b)
        return fail(PLX_ERR_INVALID, "plx_sort: key needs its second column");
    }
    if (d->nkeys > 0) hipLaunchKernelGGL(k_sort_small, dim3(1), dim3(kSortSmall), 0, s, d->n_max, d->n_dev, *d);
    return check_launch("plx_sort");
  }
  const int64_t ntiles = (d->n_max + kTile - 1) / kTile;
  int32_t* hist = d->hist;
  int32_t* scan_scratch = d->hist + 256 * ntiles;
  const bool tile_major = ntiles <= kScanTilesMax;  // each scatter scans the table itself
  for (int k = 0; k < d->nkeys; ++k) {
    const plx_sort_key& key = d->keys[k];
    if (key.bits < 1 || key.bits > 32 || !key.a) return fail(PLX_ERR_INVALID, "plx_sort: bad key");
    if ((key.kind == PLX_KEY_LEVEL_OF || key.kind == PLX_KEY_PAIR16 || key.kind == PLX_KEY_DEADMAX) && !key.b)
      return fail(PLX_ERR_INVALID, "plx_sort: key needs its second column");
    // Pass 0's histogram computes the keys from the values. With an odd
    // number of passes it also copies the values to vals_alt and pass 0
    // reads them there, so the last pass writes its order into vals.
    const int passes = (key.bits + 7) / 8;
    const bool odd = passes & 1;
    hipLaunchKernelGGL(k_radix_hist<true>, dim3(ntiles), dim3(kSortBlock), 0, s, d->n_max, d->n_dev, key, d->vals,
                       d->keys_buf, odd ? d->vals_alt : nullptr, 0, ntiles, tile_major, hist);
    uint32_t* kin = d->keys_buf;
    uint32_t* vin = odd ? d->vals_alt : d->vals;
    uint32_t* kout = d->keys_alt;
    uint32_t* vout = odd ? d->vals : d->vals_alt;
    for (int pass = 0; pass < passes; ++pass) {
      const int shift = 8 * pass;
      if (pass > 0)
        hipLaunchKernelGGL(k_radix_hist<false>, dim3(ntiles), dim3(kSortBlock), 0, s, d->n_max, d->n_dev, key,
                           nullptr, kin, nullptr, shift, ntiles, tile_major, hist);
      // (a tile-major table is scanned by the scatter itself)
      if (!tile_major) {
        const int rc = scan_or_compact(256 * ntiles, nullptr, -1, hist, hist, nullptr, scan_scratch, s, "plx_sort");
        if (rc != PLX_OK) return rc;
      }
      hipLaunchKernelGGL(k_radix_scatter, dim3(ntiles), dim3(kSortBlock), 0, s, d->n_max, d->n_dev, kin, vin, kout,
                         vout, shift, ntiles, tile_major, hist);
      uint32_t* t = kin;
      kin = kout;
      kout = t;
      t = vin;
      vin = vout;
      vout = t;
    }
  }
  return check_launch("plx_sort");
}

// ---------------------------------------------------------------------------
// Roof probes: the read bandwidth of LDS (conflict-free 16-byte reads, each
// wave reading 1 KB per instruction) and of an L2-resident buffer (16-byte
// coalesced reads of `words` uint4, a power of two, read over and over).
// Every index is masked into its buffer.
// ---------------------------------------------------------------------------
constexpr int kProbeLdsWords = 4096;  // uint4 = 64 KB
constexpr int kProbeBlocks = 2048;

__global__ __launch_bounds__(256) void k_probe_lds(uint32_t* out, int32_t iters) {
  __shared__ uint4 buf[kProbeLdsWords];
  for (int i = threadIdx.x; i < kProbeLdsWords; i += 256) buf[i] = make_uint4(i, i * 3u, i * 5u, i * 7u);
  __syncthreads();
  uint32_t acc = 0;
  int idx = threadIdx.x;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint4 v = buf[(idx + k * 256) & (kProbeLdsWords - 1)];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    idx = (idx + 64) & (kProbeLdsWords - 1);
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc;
}

__global__ __launch_bounds__(256) void k_probe_l2(const uint4* buf, int64_t words, uint32_t* out, int32_t iters) {
  uint32_t acc = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint4 v = buf[(idx + k * stride) & (words - 1)];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    idx = (idx + 8 * stride) & (words - 1);
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc;
}

int plx_grow_filter(const plx_grow_filter_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_grow_filter: null descriptor");
  if (d->n < 0 || d->num_units < 1) return fail(PLX_ERR_INVALID, "plx_grow_filter: bad sizes");
  if (d->n == 0) return PLX_OK;
  if (!d->src || !d->dst || !d->score || !d->level) return fail(PLX_ERR_INVALID, "plx_grow_filter: null column");
  if (d->nlive > 0 && (!d->live_idx || !d->live_bucket || !d->live_src || !d->live_dst))
    return fail(PLX_ERR_INVALID, "plx_grow_filter: live pair list missing");
  hipLaunchKernelGGL(k_grow_filter, dim3(grid_for(d->n)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), *d);
  return check_launch("plx_grow_filter");
}

int plx_grow_mark_repeats(int64_t n_max, const int32_t* n_dev, const int32_t* order, const int32_t* src,
                          const int32_t* dst, float* score, void* stream) {
  if (n_max < 0) return fail(PLX_ERR_INVALID, "plx_grow_mark_repeats: negative n");
  if (n_max < 2) return PLX_OK;
  if (!order || !src || !dst || !score) return fail(PLX_ERR_INVALID, "plx_grow_mark_repeats: null pointer");
  hipLaunchKernelGGL(k_mark_repeats, dim3(grid_for(n_max)), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                     n_max, n_dev, order, src, dst, score);
  return check_launch("plx_grow_mark_repeats");
}

int plx_grow_select(int64_t n_max, const int32_t* n_dev, const int32_t* sorted, const int32_t* src,
                    const int32_t* level, int32_t per_segment, int64_t k, int32_t num_segments, int32_t* first,
                    uint8_t* win, void* stream) {
  if (n_max < 0 || k < 0) return fail(PLX_ERR_INVALID, "plx_grow_select: negative size");
  if (n_max == 0) return PLX_OK;
  if (!sorted || !src || !level || !win || (per_segment && (!first || num_segments < 1)))
    return fail(PLX_ERR_INVALID, "plx_grow_select: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (per_segment)
    hipLaunchKernelGGL(k_seg_first, dim3(grid_for(n_max)), dim3(kBlock), 0, s, n_max, n_dev, sorted, src, level,
                       first);
  hipLaunchKernelGGL(k_select, dim3(grid_for(n_max)), dim3(kBlock), 0, s, n_max, n_dev, sorted, src, level,
                     per_segment, k, first, win);
  return check_launch("plx_grow_select");
}

int plx_grow_claim(const plx_grow_claim_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_grow_claim: null descriptor");
  if (d->n_max < 0 || d->ncols < 0 || d->ncols > PLX_MAX_GROW_COLS)
    return fail(PLX_ERR_INVALID, "plx_grow_claim: bad sizes");
  if (d->tail_dev && (!d->pipeline || !d->flags))
    return fail(PLX_ERR_INVALID, "plx_grow_claim: tail_dev without a PIPELINE claim's flags");
  if (d->n_max == 0) {
    if (d->tail_dev) {
      hipLaunchKernelGGL(k_claim_tail, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), d->tail_dev, d->flags);
      return check_launch("plx_grow_claim");
    }
    return PLX_OK;
  }
  if (!d->winners || !d->src || !d->dst || !d->score || !d->level || !d->from_id || !d->to_id || !d->dead ||
      !d->flags || !d->scratch)
    return fail(PLX_ERR_INVALID, "plx_grow_claim: null pointer");
  if (!d->pipeline && (!d->free_slots || !d->free_info))
    return fail(PLX_ERR_INVALID, "plx_grow_claim: free lists missing");
  if (d->pipeline && (!d->own_slots || !d->own_start || !d->own_count || d->num_levels < 1))
    return fail(PLX_ERR_INVALID, "plx_grow_claim: own-slot lists missing");
  for (int c = 0; c < d->ncols; ++c) {
    const plx_grow_col& col = d->cols[c];
    if (!col.ptr || (col.bytes != 1 && col.bytes != 4) || col.init_slot >= PLX_MAX_SOUTS ||
        (col.init_slot >= 0 && !d->init_out[col.init_slot]))
      return fail(PLX_ERR_INVALID, "plx_grow_claim: bad column");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n = d->n_max;
  int32_t* g = d->scratch;
  int32_t* g2 = g + n;
  int32_t* scan = g2 + n;
  int32_t* rank = scan + n;
  int32_t* spill = rank + n;
  int32_t* spill_rank = spill + n;
  int32_t* ss = spill_rank + 2 * n;
  const int grid = grid_for(n);
  hipLaunchKernelGGL(k_claim_growable, dim3(grid), dim3(kBlock), 0, s, *d, g);
  int32_t* grow = g;
  if (d->max_new_per_step > 0 && !d->growable_in) {
    int rc = scan_or_compact(n, d->n_dev, -1, g, scan, nullptr, ss, s, "plx_grow_claim");
    if (rc != PLX_OK) return rc;
    hipLaunchKernelGGL(k_claim_cap, dim3(grid), dim3(kBlock), 0, s, *d, g, scan, g2);
    grow = g2;
  }
  int rc = scan_or_compact(n, d->n_dev, -1, grow, scan, nullptr, ss, s, "plx_grow_claim");
  if (rc != PLX_OK) return rc;
  hipLaunchKernelGGL(k_claim_rank, dim3(grid), dim3(kBlock), 0, s, *d, grow, scan, rank, spill);
  if (d->pipeline) {
    rc = scan_or_compact(n, d->n_dev, -1, spill, spill_rank, nullptr, ss, s, "plx_grow_claim");
    if (rc != PLX_OK) return rc;
  }
  hipLaunchKernelGGL(k_claim_write, dim3(grid), dim3(kBlock), 0, s, *d, grow, rank, spill, spill_rank);
  if (d->tail_dev) hipLaunchKernelGGL(k_claim_tail, dim3(1), dim3(64), 0, s, d->tail_dev, d->flags);
  return check_launch("plx_grow_claim");
}

int plx_gather_level(int64_t n_max, const int32_t* n_dev, const int32_t* idx, const int32_t* ids,
                     const int32_t* level, int32_t bound, int32_t* out, void* stream) {
  if (n_max < 0 || bound < 1) return fail(PLX_ERR_INVALID, "plx_gather_level: bad sizes");
  if (n_max == 0) return PLX_OK;
  if (!idx || !ids || !level || !out) return fail(PLX_ERR_INVALID, "plx_gather_level: null pointer");
  hipLaunchKernelGGL(k_gather_level, dim3(grid_for(n_max)), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                     n_max, n_dev, idx, ids, level, bound, out);
  return check_launch("plx_gather_level");
}

int plx_occurrence(int64_t n, const int32_t* sorted, const int32_t* from_id, const int32_t* to_id, int32_t* occ,
                   void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_occurrence: negative n");
  if (n == 0) return PLX_OK;
  if (!sorted || !from_id || !to_id || !occ) return fail(PLX_ERR_INVALID, "plx_occurrence: null pointer");
  hipLaunchKernelGGL(k_occurrence, dim3(grid_for(n)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), n, sorted,
                     from_id, to_id, occ);
  return check_launch("plx_occurrence");
}

int plx_gather_i32(int64_t n_max, const int32_t* n_dev, const int32_t* idx, const int32_t* a, int32_t* out,
                   void* stream) {
  if (n_max < 0) return fail(PLX_ERR_INVALID, "plx_gather_i32: negative n");
  if (n_max == 0) return PLX_OK;
  if (!idx || !a || !out) return fail(PLX_ERR_INVALID, "plx_gather_i32: null pointer");
  hipLaunchKernelGGL(k_gather_i32, dim3(grid_for(n_max)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), n_max,
                     n_dev, idx, a, out);
  return check_launch("plx_gather_i32");
}

int plx_level_counts(int64_t n, const int32_t* n_dev, const int32_t* keys, int32_t nlevels, int32_t* count,
                     int32_t* start, int32_t* scratch, void* stream) {
  if (n < 0 || nlevels < 1) return fail(PLX_ERR_INVALID, "plx_level_counts: bad sizes");
  if (!count || !start || !scratch || (n > 0 && !keys))
    return fail(PLX_ERR_INVALID, "plx_level_counts: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(nlevels)), dim3(kBlock), 0, s, static_cast<int64_t>(nlevels), 0,
                     count);
  if (n > 0)
    hipLaunchKernelGGL(k_level_count, dim3(grid_for(n)), dim3(kBlock), 0, s, n, n_dev, keys, nlevels, count);
  return scan_or_compact(nlevels, nullptr, -1, count, start, nullptr, scratch, s, "plx_level_counts");
}

int plx_bucket_free(int32_t num_buckets, const int64_t* bucket_off, const int32_t* free_slots,
                    const int32_t* nfree_total, int32_t* free_info, void* stream) {
  if (num_buckets < 1) return fail(PLX_ERR_INVALID, "plx_bucket_free: no buckets");
  if (!bucket_off || !free_slots || !nfree_total || !free_info)
    return fail(PLX_ERR_INVALID, "plx_bucket_free: null pointer");
  hipLaunchKernelGGL(k_bucket_free, dim3((num_buckets + kBlock - 1) / kBlock), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), num_buckets, bucket_off, free_slots, nfree_total, free_info);
  return check_launch("plx_bucket_free");
}

int plx_mask_importance(int32_t n, const float* imp, const int32_t* level, const uint8_t* pruned, int32_t mode,
                        int32_t b, int32_t gap, int32_t direction, float* out, void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_mask_importance: negative n");
  if (n == 0) return PLX_OK;
  if (!imp || !level || !out) return fail(PLX_ERR_INVALID, "plx_mask_importance: null pointer");
  hipLaunchKernelGGL(k_mask_importance, dim3((n + kBlock - 1) / kBlock), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), n, imp, level, pruned, mode, b, gap, direction, out);
  return check_launch("plx_mask_importance");
}

int plx_unit_write(int64_t n, const int32_t* n_dev, const int32_t* idx, const uint8_t* skip, int32_t ncols,
                   const plx_unit_col* cols, const uint32_t* const* outs, void* stream) {
  if (n < 0 || !unit_cols_ok(ncols, cols)) return fail(PLX_ERR_INVALID, "plx_unit_write: bad columns");
  if (n == 0 || ncols == 0) return PLX_OK;
  if (!outs) return fail(PLX_ERR_INVALID, "plx_unit_write: null outputs");
  UnitOuts o{};
  for (int k = 0; k < ncols; ++k) {
    if (!outs[k]) return fail(PLX_ERR_INVALID, "plx_unit_write: null output");
    o.o[k] = outs[k];
  }
  hipLaunchKernelGGL(k_unit_write, dim3(grid_for(n)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), n, n_dev,
                     idx, skip, pack_cols(ncols, cols), o);
  return check_launch("plx_unit_write");
}

int plx_unit_prune(int64_t n, const uint32_t* selected, uint8_t* pruned, const uint8_t* exempt, int32_t ncols,
                   const plx_unit_col* cols, uint8_t* doomed, int32_t* doomed_count, void* stream) {
  if (n < 0 || !unit_cols_ok(ncols, cols)) return fail(PLX_ERR_INVALID, "plx_unit_prune: bad columns");
  if (n == 0) return PLX_OK;
  if (!selected || !pruned || !doomed) return fail(PLX_ERR_INVALID, "plx_unit_prune: null pointer");
  hipLaunchKernelGGL(k_unit_prune, dim3(grid_for(n)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), n, selected,
                     pruned, exempt, pack_cols(ncols, cols), doomed, doomed_count);
  return check_launch("plx_unit_prune");
}

int plx_merge_kills(int64_t n, const uint8_t* sink, uint8_t* dead, float* stamp, float stamp_value, void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_merge_kills: negative n");
  if (n == 0) return PLX_OK;
  if (!sink || !dead) return fail(PLX_ERR_INVALID, "plx_merge_kills: null pointer");
  hipLaunchKernelGGL(k_merge_kills, dim3(grid_for(n)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), n, sink,
                     dead, stamp, stamp_value);
  return check_launch("plx_merge_kills");
}

int plx_gen_fold(const plx_gen_fold_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_gen_fold: null descriptor");
  if (d->nrows < 0 || d->ncomp < 1 || d->ncomp > 8 || d->num_units <= 0 || d->batch < 1)
    return fail(PLX_ERR_INVALID, "plx_gen_fold: bad sizes (1 <= ncomp <= 8, batch >= 1)");
  if (d->nrows == 0) return PLX_OK;
  if (!d->row_unit || !d->row_ptr || (d->backward ? !d->to_id : !d->from_id))
    return fail(PLX_ERR_INVALID, "plx_gen_fold: null row table or id column");
  if (d->prog.ninstr < 0 || d->prog.ninstr > PLX_MAX_SINSTR || d->prog.nout < d->ncomp)
    return fail(PLX_ERR_INVALID, "plx_gen_fold: the program has fewer outputs than components");
  for (int k = 0; k < d->ncomp; ++k)
    if (!d->acc[k] || d->monoid[k] < PLX_MONOID_SUM || d->monoid[k] > PLX_MONOID_MIN)
      return fail(PLX_ERR_INVALID, "plx_gen_fold: bad accumulator column or monoid");
  hipLaunchKernelGGL(k_gen_fold, dim3(grid_for(d->nrows * d->batch)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), *d);
  return check_launch("plx_gen_fold");
}

int plx_kill_incident(int64_t n, const int32_t* from_id, const int32_t* to_id, uint8_t* dead, const uint8_t* doomed,
                      const int32_t* id_map, int32_t* kill_count, float* stamp, float stamp_value, void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_kill_incident: negative n");
  if (n == 0) return PLX_OK;
  if (!from_id || !to_id || !dead || !doomed) return fail(PLX_ERR_INVALID, "plx_kill_incident: null pointer");
  hipLaunchKernelGGL(k_kill_incident, dim3(grid_for(n)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), n,
                     from_id, to_id, dead, doomed, id_map, kill_count, stamp, stamp_value);
  return check_launch("plx_kill_incident");
}

int plx_sorted_starts(int64_t n, const int32_t* n_dev, const int32_t* keys, int32_t nlevels, int32_t* start,
                      void* stream) {
  if (n < 0 || n >= (int64_t{1} << 31) || nlevels < 0) return fail(PLX_ERR_INVALID, "plx_sorted_starts: bad sizes");
  if (!start || (n > 0 && !keys)) return fail(PLX_ERR_INVALID, "plx_sorted_starts: null pointer");
  hipLaunchKernelGGL(k_sorted_starts, dim3(grid_for(static_cast<int64_t>(nlevels) + 1)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), n, n_dev, keys, nlevels, start);
  return check_launch("plx_sorted_starts");
}

int plx_unit_place(int64_t n_max, const int32_t* parents, const int32_t* nparents, const int32_t* free_ids,
                   const int32_t* nfree, const int32_t* offset, int32_t* level, uint8_t* pruned, int32_t max_level,
                   int32_t ncols, const plx_unit_col* cols, int32_t* child, int32_t* parent, int32_t* flags,
                   void* stream) {
  if (n_max < 0 || max_level < 1 || !unit_cols_ok(ncols, cols))
    return fail(PLX_ERR_INVALID, "plx_unit_place: bad sizes or columns");
  if (!parents || !nparents || !free_ids || !nfree || !offset || !level || !pruned || !child || !parent || !flags)
    return fail(PLX_ERR_INVALID, "plx_unit_place: null pointer");
  hipLaunchKernelGGL(k_unit_place, dim3(grid_for(n_max > 0 ? n_max : 1)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), n_max, parents, nparents, free_ids, nfree, offset, level, pruned,
                     max_level, pack_cols(ncols, cols), child, parent, flags);
  return check_launch("plx_unit_place");
}

int plx_relax_levels(int64_t n_units, int64_t n_edges, const int32_t* from_id, const int32_t* to_id,
                     const uint8_t* dead, const int32_t* level_in, int32_t* level_out, const uint8_t* is_input,
                     int32_t* changed, void* stream) {
  if (n_units < 1 || n_edges < 0) return fail(PLX_ERR_INVALID, "plx_relax_levels: bad sizes");
  if (!level_in || !level_out || !changed || (n_edges > 0 && (!from_id || !to_id || !dead)))
    return fail(PLX_ERR_INVALID, "plx_relax_levels: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_copy_i32, dim3(grid_for(n_units)), dim3(kBlock), 0, s, n_units, level_in, level_out);
  if (n_edges > 0)
    hipLaunchKernelGGL(k_relax_edges, dim3(grid_for(n_edges)), dim3(kBlock), 0, s, n_edges, from_id, to_id, dead,
                       level_in, level_out);
  hipLaunchKernelGGL(k_pin_compare, dim3(grid_for(n_units)), dim3(kBlock), 0, s, n_units, level_in, level_out,
                     is_input, changed);
  return check_launch("plx_relax_levels");
}

int plx_resort_keys(int64_t n, const int32_t* from_id, const uint8_t* dead, const int32_t* level, int32_t pipeline,
                    int32_t sentinel, int32_t* key, void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_resort_keys: negative n");
  if (n == 0) return PLX_OK;
  if (!from_id || !dead || !level || !key) return fail(PLX_ERR_INVALID, "plx_resort_keys: null pointer");
  hipLaunchKernelGGL(k_resort_keys, dim3(grid_for(n)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), n, from_id,
                     dead, level, pipeline, sentinel, key);
  return check_launch("plx_resort_keys");
}

int plx_gather_col(int64_t n, const int32_t* n_dev, const int32_t* idx, const void* src, void* dst, int32_t bytes,
                   void* stream) {
  if (n < 0 || (bytes != 1 && bytes != 4)) return fail(PLX_ERR_INVALID, "plx_gather_col: bad size");
  if (n == 0) return PLX_OK;
  if (!idx || !src || !dst) return fail(PLX_ERR_INVALID, "plx_gather_col: null pointer");
  hipLaunchKernelGGL(k_gather_col, dim3(grid_for(n)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), n, n_dev,
                     idx, src, dst, bytes);
  return check_launch("plx_gather_col");
}

// ---------------------------------------------------------------------------
// Allocation-free ordered compaction. plx_compact_noalloc runs plx_compact's
// kernels with their chunk sums in `scratch`, a file-scope device array, so a
// caller that cannot allocate (code under stream capture, a serving loop)
// needs no workspace. Each GPU holds its own copy of the array; its address
// on a device comes from hipGetSymbolAddress, looked up once per device (the
// array's name is only a host-side handle and must never reach a kernel).
// k_chunk_sums overwrites every chunk sum a call reads, so nothing is
// cleared between calls; calls that overlap on one GPU share the array and
// race.
// ---------------------------------------------------------------------------

constexpr int64_t kNoAllocMaxN = PLX_COMPACT_NOALLOC_MAX_N;
constexpr int64_t kNoAllocInts = (kNoAllocMaxN + kChunk - 1) / kChunk;
static_assert(kNoAllocInts * kChunk >= kNoAllocMaxN, "scratch holds every chunk sum");

static __device__ __align__(256) int32_t scratch[kNoAllocInts];

namespace {

constexpr int kNoAllocDevices = 64;
std::mutex g_noalloc_mu;
int32_t* g_noalloc_ptr[kNoAllocDevices] = {};

// The current device's address of `scratch` (looked up on its first use).
int noalloc_scratch(int32_t** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return fail(PLX_ERR_HIP, "plx_compact_noalloc: hipGetDevice failed");
  if (dev < 0 || dev >= kNoAllocDevices) return fail(PLX_ERR_UNSUPPORTED, "plx_compact_noalloc: device ordinal >= 64");
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p) return fail(PLX_ERR_HIP, "plx_compact_noalloc: hipGetSymbolAddress(scratch) failed");
    g_noalloc_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_noalloc_ptr[dev];
  return PLX_OK;
}

}  // namespace

int plx_compact_noalloc(int64_t n, const int32_t* n_dev, int32_t mode, const void* flags, int32_t* out,
                        int32_t* count, void* stream) {
  if (n < 0 || mode < 0 || mode > PLX_FLAG_I32) return fail(PLX_ERR_INVALID, "plx_compact_noalloc: bad n or mode");
  if (n > kNoAllocMaxN)
    return fail(PLX_ERR_UNSUPPORTED, "plx_compact_noalloc: n exceeds PLX_COMPACT_NOALLOC_MAX_N (2^26)");
  if ((n > 0 && (!flags || !out)) || !count) return fail(PLX_ERR_INVALID, "plx_compact_noalloc: null pointer");
  int32_t* sums = nullptr;
  const int rc = noalloc_scratch(&sums);
  if (rc != PLX_OK) return rc;
  return scan_or_compact(n, n_dev, mode, flags, out, count, sums, static_cast<hipStream_t>(stream),
                         "plx_compact_noalloc");
}

int plx_roof_probe(int32_t kind, int32_t iters, const void* buf, int64_t buf_bytes, uint32_t* out, double* bytes,
                   float* ms, void* stream) {
  if (kind != PLX_PROBE_LDS && kind != PLX_PROBE_L2) return fail(PLX_ERR_INVALID, "plx_roof_probe: unknown kind");
  if (iters < 1 || !out || !bytes || !ms) return fail(PLX_ERR_INVALID, "plx_roof_probe: bad arguments");
  const int64_t words = buf_bytes / 16;
  if (kind == PLX_PROBE_L2 && (!buf || words < 1 || (words & (words - 1)) != 0))
    return fail(PLX_ERR_INVALID, "plx_roof_probe: the L2 buffer must hold a power-of-two count of 16 bytes");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess) return fail(PLX_ERR_HIP, "plx_roof_probe: event");
  if (hipEventCreate(&b) != hipSuccess) {
    (void)hipEventDestroy(a);
    return fail(PLX_ERR_HIP, "plx_roof_probe: event");
  }
  (void)hipEventRecord(a, s);
  if (kind == PLX_PROBE_LDS) {
    hipLaunchKernelGGL(k_probe_lds, dim3(kProbeBlocks), dim3(256), 0, s, out, iters);
    *bytes = double(kProbeBlocks) * 256 * iters * 16 * 16;
  } else {
    hipLaunchKernelGGL(k_probe_l2, dim3(kProbeBlocks), dim3(256), 0, s, static_cast<const uint4*>(buf), words, out,
                       iters);
    *bytes = double(kProbeBlocks) * 256 * iters * 8 * 16;
  }
  (void)hipEventRecord(b, s);
  const hipError_t e = hipEventSynchronize(b);
  float t = 0.0f;
  if (e == hipSuccess) (void)hipEventElapsedTime(&t, a, b);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  if (e != hipSuccess) return fail(PLX_ERR_HIP, "plx_roof_probe: launch failed");
  *ms = t;
  return check_launch("plx_roof_probe");
}
