// plastax_hip.hip -- gfx950 kernels of the streaming edge-arena step and the
// C ABI declared in include/plastax_hip.h.
//
// Data layout (built by plastax_amd/_layout.py): every bucket's edge columns
// live in one physical slab, destination-sorted inside each bucket (live edges
// ordered by (dst, logical slot), then the bucket's dead slots). The backward
// transpose reduce works on tiles of that order: per-(tile, source) partials,
// folded per superblock of tiles, then across superblocks. All folds
// are deterministic: no float atomics anywhere, so a step is bitwise
// repeatable.
//
// The path is a memory-bound gather / segment reduce (about 2 flops per edge
// per pass), so nothing here uses MFMA; the kernels stream the edge columns
// with 16-byte vector loads, stage per-edge terms in LDS and let each lane
// fold its own segment in slot order.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/plastax_hip.h"
#include "px_common.h"
#include "px_math.h"
#include "px_site.h"

namespace plx_detail {

thread_local std::string g_last_error;

int fail(int code, const char* what) {
  g_last_error = what;
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(err);
    return PLX_ERR_HIP;
  }
  return PLX_OK;
}

}  // namespace plx_detail

using plx_detail::check_launch;
using plx_detail::fail;

#include "px_forward.h"

namespace {

template <int M, bool PRUNE>
__global__ __launch_bounds__(kFwdBlock) void k_forward(plx_forward_desc d) {
  forward_body<M, PRUNE, SiteInterp>(d);
}

// ---------------------------------------------------------------------------
// Connection update: four physical positions per lane, 16-byte loads and
// stores of every column; dead positions store their old values back.
// ---------------------------------------------------------------------------
constexpr int kUpdBlock = 256;

template <class D>
__device__ __forceinline__ float adam_pow(const D& d, float b, float t, int which) {
  if (d.pow_table && t >= 0.0f && t < static_cast<float>(d.pow_table_len) && floorf(t) == t)
    return d.pow_table[2 * static_cast<int>(t) + which];
  return px::pow_step(b, t);
}

template <int RULE, class D>
__device__ __forceinline__ void update_one(const D& d, float grad, float& w, float& s0, float& s1,
                                           float& s2) {
  if (RULE == PLX_RULE_SGD) {
    w = w - d.p[0] * grad;
  } else if (RULE == PLX_RULE_MOMENTUM) {
    const float v = d.p[1] * s0 + grad;
    s0 = v;
    w = w - d.p[0] * v;
  } else if (RULE == PLX_RULE_ADAM) {
    const float weight = w;
    const float step = s2 + 1.0f;
    const float m = d.p[1] * s0 + d.p[5] * grad;
    const float v = d.p[2] * s1 + d.p[6] * (grad * grad);
    const float m_hat = m / (1.0f - adam_pow(d, d.p[1], step, 0));
    const float v_hat = v / (1.0f - adam_pow(d, d.p[2], step, 1));
    const float dir = m_hat / (sqrtf(v_hat) + d.p[3]);
    const float upd = d.p[0] * (dir + d.p[4] * weight);
    w = weight - upd;
    s0 = m;
    s1 = v;
    s2 = step;
  } else {  // RMSProp
    const float ms = d.p[1] * s0 + d.p[2] * (grad * grad);
    const float upd = d.p[0] * grad / sqrtf(ms + d.p[3]);
    w = w - upd;
    s0 = ms;
  }
}

// Adam with the step count shared by every live edge of the launch: the
// same float32 operations as update_one<ADAM>, with the bias-correction
// denominators 1 - b^step computed once.
template <class D>
__device__ __forceinline__ void adam_uniform(const D& d, float grad, float den1, float den2,
                                             float& w, float& m, float& v) {
  const float weight = w;
  const float mm = d.p[1] * m + d.p[5] * grad;
  const float vv = d.p[2] * v + d.p[6] * (grad * grad);
  const float m_hat = mm / den1;
  const float v_hat = vv / den2;
  const float dir = m_hat / (sqrtf(v_hat) + d.p[3]);
  const float upd = d.p[0] * (dir + d.p[4] * weight);
  w = weight - upd;
  m = mm;
  v = vv;
}

// Applies the rule to one edge: per-edge step count (state s2) or, with
// UNI_T, the launch's shared one (den1/den2 precomputed; s2 untouched).
template <int RULE, bool UNI_T, class D>
__device__ __forceinline__ void update_edge(const D& d, float grad, float den1, float den2,
                                            float& w, float& s0, float& s1, float& s2) {
  if (RULE == PLX_RULE_ADAM && UNI_T)
    adam_uniform(d, grad, den1, den2, w, s0, s1);
  else
    update_one<RULE>(d, grad, w, s0, s1, s2);
}

// Dead-byte mask of the quad at position e when the caller passes no DEAD
// column: positions at or past live_end are dead.
__device__ __forceinline__ uint32_t dead_from_end(int64_t e, int64_t live_end) {
  return (e + 0 >= live_end ? 0x000000FFu : 0u) | (e + 1 >= live_end ? 0x0000FF00u : 0u) |
         (e + 2 >= live_end ? 0x00FF0000u : 0u) | (e + 3 >= live_end ? 0xFF000000u : 0u);
}

// One 16-byte quad of positions per lane per iteration, the workgroups
// striding over the bucket (each stages its act table once). Three quads
// per lane are in flight at once: while quad e is updated, quad e + stride's
// gathers and value columns and quad e + 2 stride's addressing columns are
// loading.
template <int RULE, bool UNI_T>
__global__ __launch_bounds__(kUpdBlock) void k_update(plx_update_desc d) {
  __shared__ float tbl[kTbl];
  constexpr int nstate =
      RULE == PLX_RULE_SGD ? 0 : (RULE == PLX_RULE_ADAM ? (UNI_T ? 2 : 3) : 1);
  float den1 = 1.0f, den2 = 1.0f;
  if (RULE == PLX_RULE_ADAM && UNI_T) {
    const float step = d.step_t + 1.0f;
    den1 = 1.0f - adam_pow(d, d.p[1], step, 0);
    den2 = 1.0f - adam_pow(d, d.p[2], step, 1);
  }
  const int64_t stride = 4 * static_cast<int64_t>(gridDim.x) * kUpdBlock;
  int64_t e = 4 * (static_cast<int64_t>(blockIdx.x) * kUpdBlock + threadIdx.x);
  // Addressing columns of quad ea.
  int64_t ea = e;
  int4 sv = make_int4(0, 0, 0, 0), tv = sv;
  uint32_t dv = 0;
  // With dst8: tv.x holds the quad's four one-byte deltas and tv.y the base
  // of its 4,096-position block.
  auto load_addr = [&](int64_t at) {
    ea = at;
    if (at < d.n) {
      sv = ld_stream(d.src + at);
      if (d.dst8) {
        tv.x = static_cast<int>(ld_stream(d.dst8 + at));
        tv.y = d.blk_dst0[at >> kDst8Shift];
      } else {
        tv = ld_stream(d.dst + at);
      }
      dv = d.dead ? *reinterpret_cast<const uint32_t*>(d.dead + at) : dead_from_end(at, d.live_end);
    }
  };
  // Gathered values and value columns of the current quad.
  bool lv[4];
  float gu[4], ac[4];
  float4 w = make_float4(0.f, 0.f, 0.f, 0.f), s0 = w, s1 = w, s2 = w;
  auto gather = [&]() {
    int di[4] = {tv.x, tv.y, tv.z, tv.w};
    if (d.dst8) {
      const uint32_t dq = static_cast<uint32_t>(tv.x);
#pragma unroll
      for (int k = 0; k < 4; ++k) di[k] = tv.y + static_cast<int>((dq >> (8 * k)) & 0xFFu);
    }
    const int si[4] = {sv.x, sv.y, sv.z, sv.w};
    const bool in = ea < d.n;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lv[k] = in && !((dv >> (8 * k)) & 0xFFu);
      gu[k] = d.gfield[lv[k] ? di[k] : 0];
    }
    gather_k<4>(tbl, d.act, d.tbl_base, d.tbl_len, si, lv, ac);
  };
  auto load_vals = [&](int64_t at) {
    if (at < d.n) {
      w = ld_stream(d.weight + at);
      if (nstate >= 1) s0 = ld_stream(d.s0 + at);
      if (nstate >= 2) s1 = ld_stream(d.s1 + at);
      if (nstate >= 3) s2 = ld_stream(d.s2 + at);
    }
  };
  load_addr(e);
  stage_table<kUpdBlock>(tbl, d.act, d.tbl_base, d.tbl_len);
  __syncthreads();
  if (e >= d.n) return;
  gather();
  load_vals(e);
  load_addr(e + stride);
  for (; e < d.n; e += stride) {
    float gr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) gr[k] = gu[k] * ac[k];
    const bool l0 = lv[0], l1 = lv[1], l2 = lv[2], l3 = lv[3];
    float4 a = w, m = s0, v = s1, t = s2;
    // The next quad's gathers and loads go out before this quad's update.
    if (e + stride < d.n) {
      gather();
      load_vals(e + stride);
      load_addr(e + 2 * stride);
    }
    if (l0) update_edge<RULE, UNI_T>(d, gr[0], den1, den2, a.x, m.x, v.x, t.x);
    if (l1) update_edge<RULE, UNI_T>(d, gr[1], den1, den2, a.y, m.y, v.y, t.y);
    if (l2) update_edge<RULE, UNI_T>(d, gr[2], den1, den2, a.z, m.z, v.z, t.z);
    if (l3) update_edge<RULE, UNI_T>(d, gr[3], den1, den2, a.w, m.w, v.w, t.w);
    st_stream(d.weight + e, a);
    if (nstate >= 1) st_stream(d.s0 + e, m);
    if (nstate >= 2) st_stream(d.s1 + e, v);
    if (nstate >= 3) st_stream(d.s2 + e, t);
  }
}

// ---------------------------------------------------------------------------
// Backward + update over destination-sorted tiles; one workgroup per
// superblock (a run of consecutive tiles of near-equal total length, so every
// workgroup streams the same number of positions), walked in tile order.
//
// For each tile the workgroup streams the edge columns once (16-byte loads):
// for each live edge it forms the backward term c = weight * g[dst] with the
// pre-update weight and, when updating, applies the update rule and stores
// the new weight and optimizer state. The term goes to LDS at the edge's rank
// in the tile's (source, position) order, with a tag: the group-start bit of
// the rank and, for a hot source, its hot index. Then the tile's (source)
// groups, listed longest first in 2-byte descriptors (first rank, length),
// are folded from LDS in order, round robin over the lanes: into the
// workgroup's LDS running sum of a hot source (hot sources are the id range
// [hot_base, hot_base + nhot), so their ranks are one range of the tile and
// the tag gives the index), folded in tile order, or into the group's cold
// slot, a function of its first rank and the tile's region table. At the
// end the running hot sums are the superblock's dense row of hot_sb. No
// float atomics: every value has exactly one writer and a fixed fold order.
// ---------------------------------------------------------------------------
constexpr int kTileBlock = 512;
#ifndef PLX_TILE_QUADS
#define PLX_TILE_QUADS 2
#endif
constexpr int kTileQuads = PLX_TILE_QUADS;  // 16-byte quads per thread per streaming pass

constexpr uint32_t kRankMask = 0x0FFFu;  // sorted_rank: the rank within the tile
constexpr uint32_t kGroupStart = 0x8000u;  // sorted_rank / tag: the rank starts a group
constexpr int kTileInfo = 16;             // int32 entries of tile_info per tile
constexpr int kGrpPer = 4;                // group descriptors prefetched per thread per tile
constexpr uint32_t kLenOpen = 15;         // descriptor length field: 15 or more (the end is found)
// s_waitcnt vmcnt(0) with the other counters left alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int kWaitVmcnt0 = 0x0F70;

// The cold slot of a cold group starting at rank r of a tile, from the
// tile's info staged in LDS (tmap: [0] hlo | hhi << 16, the hot ranks;
// [1..7] the region bounds b1..b7; [8..15] the region offsets o0..o7):
// c = r less the hot ranks before it, x = the number of bounds at or below
// c, slot = o[x] + c.
__device__ __forceinline__ int cold_slot(const int32_t* tmap, int r, int hlo, int hhi) {
  const int c = r >= hhi ? r - (hhi - hlo) : r;
  int x = 0;
#pragma unroll
  for (int k = 1; k < 8; ++k) x += c >= tmap[k] ? 1 : 0;
  return tmap[8 + x] + c;
}

// Folds one (tile, source) group: the run buf[st, st + len) in order, into
// its hot running sum or its cold slot. The descriptor packs the first rank
// (low 12 bits) and the length (high 4 bits; kLenOpen: at least that long,
// the run ends at the next rank whose tag has the group-start bit, or at nr).
// A source has one group per tile, so no other lane touches a hot slot
// within the tile.
template <int M>
__device__ __forceinline__ void fold_group(const plx_tile_desc& d, const float* buf, const uint16_t* tag,
                                           float* hot, const int32_t* tmap, int hlo, int hhi, int nr,
                                           uint16_t desc) {
  const int st = desc & static_cast<int>(kRankMask);
  int len = desc >> 12;
  if (len == static_cast<int>(kLenOpen)) {
    // Eight tags per 16-byte read, from the aligned group holding st + 15.
    int j = (st + kLenOpen) & ~7;
    uint32_t skip = static_cast<uint32_t>((st + kLenOpen) & 7);  // tags of the first read before st + 15
    for (; j < nr; j += 8) {
      const uint4 g = *reinterpret_cast<const uint4*>(tag + j);
      uint32_t bits = ((g.x >> 15) & 1u) | ((g.x >> 30) & 2u) | ((g.y >> 13) & 4u) | ((g.y >> 28) & 8u) |
                      ((g.z >> 11) & 16u) | ((g.z >> 26) & 32u) | ((g.w >> 9) & 64u) | ((g.w >> 24) & 128u);
      bits &= ~((1u << skip) - 1u);
      skip = 0;
      if (bits) {
        j += __builtin_ctz(bits);
        break;
      }
    }
    len = min(j, nr) - st;
  }
  const float* run = buf + st;
  float v = Mono<M>::id();
  int j = 0;
  for (; j + 4 <= len; j += 4) {
    const float a0 = run[j], a1 = run[j + 1], a2 = run[j + 2], a3 = run[j + 3];
    v = Mono<M>::op(v, a0);
    v = Mono<M>::op(v, a1);
    v = Mono<M>::op(v, a2);
    v = Mono<M>::op(v, a3);
  }
  for (; j < len; ++j) v = Mono<M>::op(v, run[j]);
  if (st >= hlo && st < hhi) {
    const int h = tag[st] & 0x7FFF;
    hot[h] = Mono<M>::op(hot[h], v);
  } else {
    d.cold_partial[cold_slot(tmap, st, hlo, hhi)] = v;
  }
}

// SAME_G: the backward field and the update's grad field are one column, so
// one gather serves both.
// SAME_G: the backward field and the update's grad field are one column, so
// one gather serves both. FAST: the layout has one-byte destinations and the
// caller passes no DEAD column (the common case), so neither is a branch at
// run time.
template <int RULE, int M, bool FOLD, bool SAME_G, bool UNI_T, bool FAST>
__global__ __launch_bounds__(kTileBlock, 2) void k_tile(plx_tile_desc d) {
  // Known at compile time on the FAST path: one-byte destinations, no DEAD.
  const bool dst8 = FAST || d.dst8 != nullptr;
  const bool dead = !FAST && d.dead != nullptr;
  extern __shared__ __align__(16) unsigned char smem[];
  const int T = d.tile_size;
  float* buf = reinterpret_cast<float*>(smem);  // [T] terms in source-sorted order
  // [T] rank tags: group-start bit | hot index (hot sources)
  uint16_t* tag = reinterpret_cast<uint16_t*>(smem + 4 * T);
  // [kTileInfo] the folded tile's info
  int32_t* tmap = reinterpret_cast<int32_t*>(smem + 4 * T + ((2 * T + 15) & ~15));
  float* hot = reinterpret_cast<float*>(tmap + kTileInfo);  // [nhot]
  // [tbl_len] act of the busiest sources (the whole allocation without fold)
  float* tbl = FOLD ? hot + ((d.nhot + 3) & ~3) : reinterpret_cast<float*>(smem);
  const int k0 = ld_uniform(d.super_tile, blockIdx.x);
  const int k1 = ld_uniform(d.super_tile, blockIdx.x + 1);
  const float ident = Mono<M>::id();
  constexpr int nstate = RULE < 0 || RULE == PLX_RULE_SGD
                             ? 0
                             : (RULE == PLX_RULE_ADAM ? (UNI_T ? 2 : 3) : 1);
  float den1 = 1.0f, den2 = 1.0f;
  if (RULE == PLX_RULE_ADAM && UNI_T) {
    const float step = d.step_t + 1.0f;
    den1 = 1.0f - adam_pow(d, d.p[1], step, 0);
    den2 = 1.0f - adam_pow(d, d.p[2], step, 1);
  }
  constexpr int U = kTileQuads;  // a tile is one pass: at most 4 * U * kTileBlock positions

  // The pipeline runs three tiles at once. While tile blk is folded from
  // LDS, tile blk + 1's gathers (g[dst], act[src]) and value columns
  // (weight, optimizer state, sorted rank, tile info) are in flight, and so
  // are tile blk + 2's addressing columns (dst, src, dead), which the
  // gathers of the next iteration need.
  int4 sv[U], tv[U];  // addressing columns of tile `an` (the next to gather)
  // Dead bytes of those quads: dl from DEAD, de from live_end (the other
  // one 0). Loaded columns and computed values never share a register (nor
  // do the two TO_ID forms, tv and t8): a register written on one path and
  // loaded on the other would make every path wait for all memory
  // operations in flight.
  uint32_t dl[U], de[U], t8[U];
  int64_t ta = 0;
  int na = 0;
  // With dst8, a position's TO_ID is the first destination of its 4,096-
  // position block plus a one-byte delta (positions are destination-sorted):
  // t8[i] holds the quad's four deltas; a tile spans at most two blocks,
  // whose bases are ad_lo and ad_hi.
  int ab_lo = 0, ad_lo = 0, ad_hi = 0;
  auto load_addr = [&](int blk) {
    const int p0 = ld_uniform(d.tile_pos, blk), p1 = ld_uniform(d.tile_pos, blk + 1);
    ta = d.base + p0;
    na = p1 - p0;
    if (dst8) {
      ab_lo = p0 >> kDst8Shift;
      ad_lo = ld_uniform(d.blk_dst0, ab_lo);
      ad_hi = ld_uniform(d.blk_dst0, (p1 - 1) >> kDst8Shift);
    }
    if (na <= 0) return;  // (tiles are never empty; uniform)
#pragma unroll
    for (int i = 0; i < U; ++i) {
      // Lanes past the tile's end load its last quad again (one more
      // request to a line already read; gather() marks them out of the
      // tile), so no load is under a lane-dependent branch, and each
      // register is cleared before the uniform branches that may load it:
      // merging a loaded register with an older value would wait for every
      // memory operation in flight.
      const int q = min(static_cast<int>(threadIdx.x) + i * kTileBlock, (na >> 2) - 1);
      const int64_t e = ta + 4 * q;
      t8[i] = 0u;
      tv[i] = make_int4(0, 0, 0, 0);
      dl[i] = 0u;
      if (dst8)
        t8[i] = ld_stream(d.dst8 + (e - d.base));
      else
        tv[i] = ld_stream(d.dst + e);
      if (RULE >= 0 || FOLD) sv[i] = ld_stream(d.src + e);
      if (dead) dl[i] = *reinterpret_cast<const uint32_t*>(d.dead + e);
      de[i] = dead ? 0u : dead_from_end(e, d.live_end);
    }
  };
  // Value columns and gathered values of the current tile.
  uint2 rk[U];
  float4 w[U], s0[U], s1[U], s2[U];
  bool lv[U][4];
  float gd[U][4], gu[U][4];
  uint32_t ah[U][4], am[U][4];  // act gathers: table hits, misses (gather_join)
  int64_t t0 = 0;
  int n = 0;
  uint32_t ht[U][2];  // hot tags of the gathered tile: src - hot_base (hot sources), else 0
  int32_t tiv = 0;  // lane k < kTileInfo: entry k of the info of the tile whose values are loaded
  uint16_t gdesc[kGrpPer];  // group descriptors of that tile (this thread's share)
  int ga = 0, gb = 0;
  // Gathers of the tile whose addressing columns are in registers; every one
  // is issued before any result is used (dead or out-of-tile lanes gather a
  // harmless unit).
  auto gather = [&]() {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const bool in = 4 * (threadIdx.x + i * kTileBlock) < na;
      int di[4] = {tv[i].x, tv[i].y, tv[i].z, tv[i].w};
      if (dst8) {
        const uint32_t dq = t8[i];
        const int rel = static_cast<int>(ta - d.base) + 4 * (static_cast<int>(threadIdx.x) + i * kTileBlock);
        const int d0 = (rel >> kDst8Shift) == ab_lo ? ad_lo : ad_hi;
#pragma unroll
        for (int k = 0; k < 4; ++k) di[k] = d0 + static_cast<int>((dq >> (8 * k)) & 0xFFu);
      }
      const int si[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        lv[i][k] = in && !(((dl[i] | de[i]) >> (8 * k)) & 0xFFu);
        const int dk = lv[i][k] ? di[k] : 0;
        if (FOLD) gd[i][k] = d.g[dk];
        if (RULE >= 0) gu[i][k] = SAME_G && FOLD ? 0.0f : d.gfield[dk];
      }
      if (RULE >= 0) gather_split<4>(tbl, d.act, d.tbl_base, d.tbl_len, si, lv[i], ah[i], am[i]);
      if (FOLD) {
        uint32_t h[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t o = static_cast<uint32_t>(si[k] - d.hot_base);
          h[k] = o < static_cast<uint32_t>(d.nhot) ? o : 0u;
        }
        ht[i][0] = h[0] | (h[1] << 16);
        ht[i][1] = h[2] | (h[3] << 16);
      }
    }
    t0 = ta;
    n = na;
  };
  // Value columns and tile info of tile blk (positions t0.., n).
  auto load_vals = [&](int blk) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      // As in load_addr: lanes past the tile's end load its last quad (the
      // update loop skips them; tiles are never empty).
      const int q = max(min(static_cast<int>(threadIdx.x) + i * kTileBlock, (n >> 2) - 1), 0);
      const int64_t e = t0 + 4 * q;
      w[i] = ld_stream(d.weight + e);
      if (FOLD) rk[i] = ld_stream(d.sorted_rank + (e - d.base));
      if (nstate >= 1) s0[i] = ld_stream(d.s0 + e);
      if (nstate >= 2) s1[i] = ld_stream(d.s1 + e);
      if (nstate >= 3) s2[i] = ld_stream(d.s2 + e);
    }
    if (FOLD) {
      // Every lane loads an entry (lanes past kTileInfo repeat the first
      // ones: one cache line), so the load is not under a branch.
      tiv = d.tile_info[static_cast<int64_t>(blk) * kTileInfo + (threadIdx.x & (kTileInfo - 1))];
      ga = ld_uniform(d.grp_off, blk);
      gb = ld_uniform(d.grp_off, blk + 1);
#pragma unroll
      for (int i = 0; i < kGrpPer; ++i) {
        const int gi = ga + threadIdx.x + i * kTileBlock;
        if (gi < gb) gdesc[i] = d.grp[gi];
      }
    }
  };

  load_addr(k0);
  if (RULE >= 0) stage_table<kTileBlock>(tbl, d.act, d.tbl_base, d.tbl_len);
  if (FOLD)
    for (int j = threadIdx.x; j < d.nhot; j += kTileBlock) hot[j] = ident;
  __syncthreads();
  gather();
  load_vals(k0);
  if (k0 + 1 < k1) load_addr(k0 + 1);
  for (int blk = k0; blk < k1; ++blk) {
    // Every load issued for this tile and the next tile's addressing columns
    // is waited for here, before this tile's stores: the memory counter
    // retires in order, so a wait for the addressing columns after the
    // stores would wait for the stores too. This tile's info and group
    // descriptors are taken here for the same reason. (The previous tile's
    // fold, which read tmap, ended at a barrier.)
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    if (FOLD && threadIdx.x < kTileInfo) tmap[threadIdx.x] = tiv;
    uint16_t cgd[kGrpPer];
    const int cga = ga, cgb = gb;
#pragma unroll
    for (int i = 0; i < kGrpPer; ++i) cgd[i] = gdesc[i];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int q = threadIdx.x + i * kTileBlock;
      if (4 * q >= n) continue;
      const int64_t e = t0 + 4 * q;
      if (FOLD) {
        // Each live edge's term goes to its rank in the tile's (source,
        // position) order, so every (tile, source) group is a contiguous run
        // of buf, and its tag to the same rank. A position tombstoned after
        // the layout was built (below live_end) keeps its rank and tag and
        // contributes the identity; every group folds from the identity, so
        // that leaves the fold's bits unchanged.
        const uint32_t rw[4] = {rk[i].x & 0xFFFFu, rk[i].x >> 16, rk[i].y & 0xFFFFu, rk[i].y >> 16};
        const uint32_t hw[4] = {ht[i][0] & 0xFFFFu, ht[i][0] >> 16, ht[i][1] & 0xFFFFu, ht[i][1] >> 16};
        const float wk[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (lv[i][k] || e + k < d.live_end) {
            const uint32_t r = rw[k] & kRankMask;
            buf[r] = lv[i][k] ? map_term(d.map, wk[k], gd[i][k]) : ident;
            tag[r] = static_cast<uint16_t>((rw[k] & kGroupStart) | hw[k]);
          }
        }
      }
      if (RULE >= 0) {
        float gr[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
          gr[k] = (SAME_G && FOLD ? gd[i][k] : gu[i][k]) * gather_join(ah[i][k], am[i][k]);
        float4 a = w[i], m = s0[i], v = s1[i], t = s2[i];
        if (lv[i][0]) update_edge<RULE, UNI_T>(d, gr[0], den1, den2, a.x, m.x, v.x, t.x);
        if (lv[i][1]) update_edge<RULE, UNI_T>(d, gr[1], den1, den2, a.y, m.y, v.y, t.y);
        if (lv[i][2]) update_edge<RULE, UNI_T>(d, gr[2], den1, den2, a.z, m.z, v.z, t.z);
        if (lv[i][3]) update_edge<RULE, UNI_T>(d, gr[3], den1, den2, a.w, m.w, v.w, t.w);
        st_stream(d.weight + e, a);
        if (nstate >= 1) st_stream(d.s0 + e, m);
        if (nstate >= 2) st_stream(d.s1 + e, v);
        if (nstate >= 3) st_stream(d.s2 + e, t);
      }
    }
    // This tile's ranked length, kept while the next tile loads.
    const int nr = static_cast<int>(max(static_cast<int64_t>(0), min(static_cast<int64_t>(n), d.live_end - t0)));
    if (blk + 1 < k1) {
      gather();
      load_vals(blk + 1);
      if (blk + 2 < k1) load_addr(blk + 2);
    }
    if (!FOLD) continue;
    __syncthreads();
    const int hlo = tmap[0] & 0xFFFF, hhi = tmap[0] >> 16;
#pragma unroll
    for (int i = 0; i < kGrpPer; ++i) {
      const int gi = cga + threadIdx.x + i * kTileBlock;
      if (gi < cgb) fold_group<M>(d, buf, tag, hot, tmap, hlo, hhi, nr, cgd[i]);
    }
    // Tiles with more groups than the prefetch covers fold the rest here.
    for (int gi = cga + kGrpPer * kTileBlock + threadIdx.x; gi < cgb; gi += kTileBlock)
      fold_group<M>(d, buf, tag, hot, tmap, hlo, hhi, nr, d.grp[gi]);
    __syncthreads();
  }
  if (!FOLD) return;
  float* hp = d.hot_sb + static_cast<int64_t>(blockIdx.x) * d.nhot;
  for (int j = threadIdx.x; j < d.nhot; j += kTileBlock) hp[j] = hot[j];
}

// Backward finalize of one row: combine its sum into acc and, where the row
// finalizes, run the apply program and reset acc.
template <int M>
__device__ __forceinline__ void finish_row(const plx_partials_desc& d, const RowPre& pre, float s) {
  const int u = pre.u;
  const float a = Mono<M>::op(d.acc ? d.acc[u] : Mono<M>::id(), s);
  if (pre.fin) {
    run_program(d.apply, u, pre.f, a, 0.0f, true);
    if (d.acc) d.acc[u] = Mono<M>::id();
  } else if (d.acc) {
    d.acc[u] = a;
  }
}

// Backward finalize of one level, one launch: the first hot_wgs workgroups
// take the hot rows, kHotCols columns each, the rest the cold rows.
//
// Hot rows (rows [0, nhot) are hot columns 0..nhot-1 in order): the
// workgroup stages its columns of hot_sb through LDS, kHotSbChunk
// superblocks at a time, with coalesced loads, and each column's lane folds
// its superblock sums in order.
//
// Cold rows: part k is rows [part_rows[k], part_rows[k+1]) (at most
// kPartBlock, one per lane, cut so that their cold runs mostly fit one
// window); hot column blocks and cold parts go to the workgroups by
// xcd_item, so each XCD takes a contiguous range of each. A workgroup's rows own one contiguous range of the source-major
// cold arrays, which is staged through LDS with coalesced loads; each row
// folds its run in tile order, closing a superblock sum whenever the
// superblock id changes.
#ifndef PLX_HOT_COLS
#define PLX_HOT_COLS 16
#endif
#ifndef PLX_HOT_CHUNK
#define PLX_HOT_CHUNK 256
#endif
constexpr int kFinBlock = 256;
constexpr int kHotCols = PLX_HOT_COLS;
constexpr int kHotSbChunk = PLX_HOT_CHUNK;
constexpr int kPartBlock = kFinBlock;
constexpr int kPartWin = 2048;
constexpr size_t kFinLds = (kHotSbChunk * kHotCols * 4 > kPartWin * 6) ? kHotSbChunk * kHotCols * 4
                                                                       : kPartWin * 6;

// Workgroup w of a launch runs on XCD w % 8. Of the n consecutive
// workgroups from `first`, the i-th takes item xcd_item(first, i, n): the
// items of each XCD are one contiguous range, XCD 0's first, so an XCD's
// workgroups read neighbouring data (one L2 per XCD).
__device__ __forceinline__ int xcd_item(int first, int i, int n) {
  const int x = (first + i) & 7;
  int p = 0;
  for (int y = 0; y < x; ++y) {
    const int r = (y - first) & 7;  // the first i with (first + i) % 8 == y
    p += r < n ? (n - r + 7) >> 3 : 0;
  }
  return p + (i >> 3);
}

template <int M>
__device__ __forceinline__ void finalize_hot(const plx_partials_desc& d, float* stage, int wg) {
  const int c0 = wg * kHotCols;
  const int ncol = min(kHotCols, d.nhot - c0);
  const bool has = static_cast<int>(threadIdx.x) < ncol;
  RowPre pre;
  if (has) pre = prefetch_row(d.row_unit, c0 + threadIdx.x, d.fin, d.apply);
  float s = Mono<M>::id();
  constexpr int kPer = kHotSbChunk * kHotCols / kFinBlock;  // staged values per thread
  for (int sb0 = 0; sb0 < d.nsuper; sb0 += kHotSbChunk) {
    const int nsb = min(kHotSbChunk, d.nsuper - sb0);
    // Issue every load of the chunk before storing any of it.
    float v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int j = threadIdx.x + i * kFinBlock;
      // Clamped into range: every load is unconditional (values past the
      // chunk are staged but never folded).
      const int sb = min(j / kHotCols, nsb - 1), c = min(j % kHotCols, ncol - 1);
      v[i] = d.hot_sb[static_cast<int64_t>(sb0 + sb) * d.nhot + c0 + c];
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) stage[threadIdx.x + i * kFinBlock] = v[i];
    __syncthreads();
    if (has) {
      // Eight LDS reads in flight per step of the (sequential) fold.
      const float* col = stage + threadIdx.x;
      int sb = 0;
      for (; sb + 8 <= nsb; sb += 8) {
        float x[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = col[(sb + k) * kHotCols];
#pragma unroll
        for (int k = 0; k < 8; ++k) s = Mono<M>::op(s, x[k]);
      }
      for (; sb < nsb; ++sb) s = Mono<M>::op(s, col[sb * kHotCols]);
    }
    __syncthreads();
  }
  if (has) finish_row<M>(d, pre, s);
}

template <int M>
__device__ __forceinline__ void finalize_cold(const plx_partials_desc& d, float* cval,
                                              uint16_t* csb, int wg) {
  int row0, rend, c_first = 0, c_last = 0;
  if (d.part_info) {
    // One load gives the rows and their cold range, so the window's loads
    // need not wait for row_cold.
    const int4 pi = reinterpret_cast<const int4*>(d.part_info)[wg];
    row0 = pi.x;
    rend = pi.y;
    c_first = pi.z;
    c_last = pi.w;
  } else {
    row0 = d.part_rows[wg];
    rend = d.part_rows[wg + 1];
  }
  const int r = row0 + static_cast<int>(threadIdx.x);
  const bool has = r < rend;
  RowPre pre;
  if (has) pre = prefetch_row(d.row_unit, r, d.fin, d.apply);
  const float ident = Mono<M>::id();
  float s = ident;
  if (d.row_cold) {
    const int c_begin = d.part_info ? c_first : d.row_cold[row0];
    const int c_end = d.part_info ? c_last : d.row_cold[rend];
    const int j0 = has ? d.row_cold[r] : 0;
    const int j1 = has ? d.row_cold[r + 1] : 0;
    float q = ident;
    int cur = -1;
    for (int w0 = c_begin; w0 < c_end; w0 += kPartWin) {
      const int wn = min(kPartWin, c_end - w0);
      // Issue every load of the window before storing any of it: the
      // window's slots and superblock ids, then the partials they name.
      constexpr int kPer = kPartWin / kPartBlock;
      int pi[kPer];
      float pv[kPer];
      uint16_t ps[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        // Clamped into range: every load is unconditional (entries past the
        // window are staged but never folded).
        const int j = min(static_cast<int>(threadIdx.x) + i * kPartBlock, wn - 1);
        pi[i] = d.cold_idx[w0 + j];
        ps[i] = d.cold_sb[w0 + j];
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) pv[i] = d.cold_partial[pi[i]];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        cval[threadIdx.x + i * kPartBlock] = pv[i];
        csb[threadIdx.x + i * kPartBlock] = ps[i];
      }
      __syncthreads();
      const int lo = max(j0, w0), hi = min(j1, w0 + wn);
      // Eight entries' LDS reads in flight per step of the fold.
      int j = lo;
      for (; j + 8 <= hi; j += 8) {
        float x[8];
        int b[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          x[k] = cval[j + k - w0];
          b[k] = csb[j + k - w0];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if (b[k] != cur) {
            if (cur >= 0) s = Mono<M>::op(s, q);
            q = ident;
            cur = b[k];
          }
          q = Mono<M>::op(q, x[k]);
        }
      }
      for (; j < hi; ++j) {
        const int sb = csb[j - w0];
        if (sb != cur) {
          if (cur >= 0) s = Mono<M>::op(s, q);
          q = ident;
          cur = sb;
        }
        q = Mono<M>::op(q, cval[j - w0]);
      }
      __syncthreads();
    }
    if (cur >= 0) s = Mono<M>::op(s, q);
  }
  if (has) finish_row<M>(d, pre, s);
}

template <int M>
__global__ __launch_bounds__(kFinBlock) void k_finalize(plx_partials_desc d, int hot_wgs) {
  __shared__ __align__(16) unsigned char smem[kFinLds];
  const int wg = static_cast<int>(blockIdx.x);
  if (wg < hot_wgs) {
    finalize_hot<M>(d, reinterpret_cast<float*>(smem), xcd_item(0, wg, hot_wgs));
  } else {
    float* cval = reinterpret_cast<float*>(smem);
    uint16_t* csb = reinterpret_cast<uint16_t*>(smem + kPartWin * 4);
    finalize_cold<M>(d, cval, csb, xcd_item(hot_wgs, wg - hot_wgs, d.nparts));
  }
}

// ---------------------------------------------------------------------------
// Batched steps. Unit columns are [num_units][B]: a row of the forward or
// the backward is one workgroup whose lanes are the samples, so the gathered
// unit row (x[src * B ..] or g[dst * B ..]) is one coalesced B-wide read,
// while FROM_ID / TO_ID / WEIGHT / DEAD are uniform across the workgroup.
// Each lane folds its sample's terms in the streaming step's order.
// ---------------------------------------------------------------------------
constexpr int kBatchBlock = 256;
constexpr int kBatchUnroll = 8;       // positions whose loads are in flight together (one wave per row)
constexpr int kBatchUnrollWide = 16;  // the same for a 256-lane workgroup per row (levels of few, long rows)

// Combines a row's sum into acc and finalizes it for sample lane `idx`.
template <int M>
__device__ __forceinline__ void finish_batch(float* acc, const plx_program& P, bool fin, int64_t idx,
                                             float s) {
  const float a = Mono<M>::op(acc ? acc[idx] : Mono<M>::id(), s);
  if (fin) {
    run_program(P, idx, load_fields(P, idx), a, 0.0f, true);
    if (acc) acc[idx] = Mono<M>::id();
  } else if (acc) {
    acc[idx] = a;
  }
}

template <int M>
__global__ __launch_bounds__(kBatchBlock) void k_forward_batch(plx_forward_desc d, int32_t B) {
  const int r = blockIdx.x;
  const int u = d.row_unit[r];
  const int e0 = d.row_ptr[r], e1 = d.row_ptr[r + 1];
  const bool fin = finalizes(d.fin, u);
  const float ident = Mono<M>::id();
  for (int b0 = 0; b0 < B; b0 += blockDim.x) {
    const int b = b0 + static_cast<int>(threadIdx.x);
    const int bl = b < B ? b : B - 1;  // every lane's loads stay in its row
    float s = ident;
    int e = e0;
    for (; e + kBatchUnrollWide <= e1; e += kBatchUnrollWide) {
      int sv[kBatchUnrollWide];
      float wv[kBatchUnrollWide], xv[kBatchUnrollWide];
      bool live[kBatchUnrollWide];
#pragma unroll
      for (int k = 0; k < kBatchUnrollWide; ++k) {
        sv[k] = d.src[e + k];
        wv[k] = d.weight[e + k];
        live[k] = d.dead ? d.dead[e + k] == 0 : true;
      }
#pragma unroll
      for (int k = 0; k < kBatchUnrollWide; ++k) xv[k] = d.x[static_cast<int64_t>(sv[k]) * B + bl];
#pragma unroll
      for (int k = 0; k < kBatchUnrollWide; ++k)
        if (live[k]) s = Mono<M>::op(s, map_term(d.map, wv[k], xv[k]));
    }
    for (; e < e1; ++e) {
      if (d.dead && d.dead[e]) continue;
      s = Mono<M>::op(s, map_term(d.map, d.weight[e], d.x[static_cast<int64_t>(d.src[e]) * B + bl]));
    }
    if (b < B) finish_batch<M>(d.acc, d.apply, fin, static_cast<int64_t>(u) * B + b, s);
  }
}

// The same forward with one wave per row and four samples per lane (16-byte
// loads of the gathered rows; B a multiple of 4): each sample's fold is the
// row's positions in order, as above.
template <int M>
__global__ __launch_bounds__(64) void k_forward_batch4(plx_forward_desc d, int32_t B) {
  const int r = blockIdx.x;
  const int u = d.row_unit[r];
  const int e0 = d.row_ptr[r], e1 = d.row_ptr[r + 1];
  const bool fin = finalizes(d.fin, u);
  const float ident = Mono<M>::id();
  for (int b0 = 0; b0 < B; b0 += 256) {
    const int b = b0 + 4 * static_cast<int>(threadIdx.x);
    const int bl = b < B ? b : B - 4;  // every lane's loads stay in its row
    float s[4] = {ident, ident, ident, ident};
    int e = e0;
    for (; e + kBatchUnroll <= e1; e += kBatchUnroll) {
      int sv[kBatchUnroll];
      float wv[kBatchUnroll];
      bool live[kBatchUnroll];
      float4 xv[kBatchUnroll];
#pragma unroll
      for (int k = 0; k < kBatchUnroll; ++k) {
        sv[k] = d.src[e + k];
        wv[k] = d.weight[e + k];
        live[k] = d.dead ? d.dead[e + k] == 0 : true;
      }
#pragma unroll
      for (int k = 0; k < kBatchUnroll; ++k)
        xv[k] = *reinterpret_cast<const float4*>(d.x + static_cast<int64_t>(sv[k]) * B + bl);
#pragma unroll
      for (int k = 0; k < kBatchUnroll; ++k) {
        if (!live[k]) continue;
        s[0] = Mono<M>::op(s[0], map_term(d.map, wv[k], xv[k].x));
        s[1] = Mono<M>::op(s[1], map_term(d.map, wv[k], xv[k].y));
        s[2] = Mono<M>::op(s[2], map_term(d.map, wv[k], xv[k].z));
        s[3] = Mono<M>::op(s[3], map_term(d.map, wv[k], xv[k].w));
      }
    }
    for (; e < e1; ++e) {
      if (d.dead && d.dead[e]) continue;
      const float w = d.weight[e];
      const float4 x = *reinterpret_cast<const float4*>(d.x + static_cast<int64_t>(d.src[e]) * B + bl);
      s[0] = Mono<M>::op(s[0], map_term(d.map, w, x.x));
      s[1] = Mono<M>::op(s[1], map_term(d.map, w, x.y));
      s[2] = Mono<M>::op(s[2], map_term(d.map, w, x.z));
      s[3] = Mono<M>::op(s[3], map_term(d.map, w, x.w));
    }
    if (b < B)
#pragma unroll
      for (int k = 0; k < 4; ++k) finish_batch<M>(d.acc, d.apply, fin, static_cast<int64_t>(u) * B + b + k, s[k]);
  }
}

template <int M>
__global__ __launch_bounds__(kBatchBlock) void k_backward_batch(plx_bwd_batch_desc d) {
  const int r = blockIdx.x;
  const int B = d.batch;
  const int u = d.row_unit[r];
  const int j0 = d.row_ptr[r], j1 = d.row_ptr[r + 1];
  const bool fin = finalizes(d.fin, u);
  const float ident = Mono<M>::id();
  for (int b0 = 0; b0 < B; b0 += blockDim.x) {
    const int b = b0 + static_cast<int>(threadIdx.x);
    const int bl = b < B ? b : B - 1;
    float s = ident;
    int j = j0;
    for (; j + kBatchUnrollWide <= j1; j += kBatchUnrollWide) {
      int tv[kBatchUnrollWide];
      float wv[kBatchUnrollWide], gv[kBatchUnrollWide];
      bool live[kBatchUnrollWide];
#pragma unroll
      for (int k = 0; k < kBatchUnrollWide; ++k) {
        tv[k] = d.dst[j + k];
        wv[k] = d.weight[j + k];
        live[k] = d.live ? d.live[j + k] != 0 : true;
      }
#pragma unroll
      for (int k = 0; k < kBatchUnrollWide; ++k) gv[k] = d.g[static_cast<int64_t>(tv[k]) * B + bl];
#pragma unroll
      for (int k = 0; k < kBatchUnrollWide; ++k)
        if (live[k]) s = Mono<M>::op(s, map_term(d.map, wv[k], gv[k]));
    }
    for (; j < j1; ++j) {
      if (d.live && !d.live[j]) continue;
      s = Mono<M>::op(s, map_term(d.map, d.weight[j], d.g[static_cast<int64_t>(d.dst[j]) * B + bl]));
    }
    if (b < B) finish_batch<M>(d.acc, d.apply, fin, static_cast<int64_t>(u) * B + b, s);
  }
}

// The same backward with one wave per row and four samples per lane
// (16-byte loads of the gathered g rows; B a multiple of 4).
template <int M>
__global__ __launch_bounds__(64) void k_backward_batch4(plx_bwd_batch_desc d) {
  const int r = blockIdx.x;
  const int B = d.batch;
  const int u = d.row_unit[r];
  const int j0 = d.row_ptr[r], j1 = d.row_ptr[r + 1];
  const bool fin = finalizes(d.fin, u);
  const float ident = Mono<M>::id();
  for (int b0 = 0; b0 < B; b0 += 256) {
    const int b = b0 + 4 * static_cast<int>(threadIdx.x);
    const int bl = b < B ? b : B - 4;
    float s[4] = {ident, ident, ident, ident};
    int j = j0;
    for (; j + kBatchUnroll <= j1; j += kBatchUnroll) {
      int tv[kBatchUnroll];
      float wv[kBatchUnroll];
      bool live[kBatchUnroll];
      float4 gv[kBatchUnroll];
#pragma unroll
      for (int k = 0; k < kBatchUnroll; ++k) {
        tv[k] = d.dst[j + k];
        wv[k] = d.weight[j + k];
        live[k] = d.live ? d.live[j + k] != 0 : true;
      }
#pragma unroll
      for (int k = 0; k < kBatchUnroll; ++k)
        gv[k] = *reinterpret_cast<const float4*>(d.g + static_cast<int64_t>(tv[k]) * B + bl);
#pragma unroll
      for (int k = 0; k < kBatchUnroll; ++k) {
        if (!live[k]) continue;
        s[0] = Mono<M>::op(s[0], map_term(d.map, wv[k], gv[k].x));
        s[1] = Mono<M>::op(s[1], map_term(d.map, wv[k], gv[k].y));
        s[2] = Mono<M>::op(s[2], map_term(d.map, wv[k], gv[k].z));
        s[3] = Mono<M>::op(s[3], map_term(d.map, wv[k], gv[k].w));
      }
    }
    for (; j < j1; ++j) {
      if (d.live && !d.live[j]) continue;
      const float w = d.weight[j];
      const float4 g = *reinterpret_cast<const float4*>(d.g + static_cast<int64_t>(d.dst[j]) * B + bl);
      s[0] = Mono<M>::op(s[0], map_term(d.map, w, g.x));
      s[1] = Mono<M>::op(s[1], map_term(d.map, w, g.y));
      s[2] = Mono<M>::op(s[2], map_term(d.map, w, g.z));
      s[3] = Mono<M>::op(s[3], map_term(d.map, w, g.w));
    }
    if (b < B)
#pragma unroll
      for (int k = 0; k < 4; ++k) finish_batch<M>(d.acc, d.apply, fin, static_cast<int64_t>(u) * B + b + k, s[k]);
  }
}

// Streaming backward over slot-ordered lists: lane = row (source unit),
// folding its list in order from the identity, then the finalize.
template <int M>
__global__ __launch_bounds__(kBatchBlock) void k_backward_lists(plx_bwd_batch_desc d) {
  const int r = blockIdx.x * kBatchBlock + threadIdx.x;
  if (r >= d.nrows) return;
  const int u = d.row_unit[r];
  const int j0 = d.row_ptr[r], j1 = d.row_ptr[r + 1];
  RowPre pre = prefetch_row(d.row_unit, r, d.fin, d.apply);
  // A constant factor of the map is not loaded (uniform branches): a count
  // pass (both factors constant) reads only liveness, or nothing.
  const bool need_w = !(d.map.flags & PLX_MAP_W_CONST);
  const bool need_x = !(d.map.flags & PLX_MAP_X_CONST);
  float s = Mono<M>::id();
  int j = j0;
  for (; j + 4 <= j1; j += 4) {
    int tv[4];
    float wv[4], gv[4];
    bool live[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      tv[k] = need_x ? d.dst[j + k] : 0;
      wv[k] = need_w ? d.weight[j + k] : 0.0f;
      live[k] = d.live ? d.live[j + k] != 0 : true;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) gv[k] = need_x ? d.g[tv[k]] : 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (live[k]) s = Mono<M>::op(s, map_term(d.map, wv[k], gv[k]));
  }
  for (; j < j1; ++j) {
    if (d.live && !d.live[j]) continue;
    s = Mono<M>::op(s, map_term(d.map, need_w ? d.weight[j] : 0.0f, need_x ? d.g[d.dst[j]] : 0.0f));
  }
  const float a = Mono<M>::op(d.acc ? d.acc[u] : Mono<M>::id(), s);
  if (pre.fin) {
    run_program(d.apply, u, pre.f, a, 0.0f, true);
    if (d.acc) d.acc[u] = Mono<M>::id();
  } else if (d.acc) {
    d.acc[u] = a;
  }
}

__global__ void k_gather_edges(int64_t n, const int32_t* pos, const float* weight, const uint8_t* dead,
                               float* out_w, uint8_t* out_live) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int p = pos[j];
  if (out_w) out_w[j] = weight[p];
  if (out_live) out_live[j] = dead ? (dead[p] == 0) : 1;
}

// The batched update, one lane per position: its batch-mean gradient is
// stat_0 + stat_1 + ... in sample order, / B (phases.py:462-471), with
// stat_b = gfield[dst * B + b] * act[src * B + b], then the update rule.
// The two B-wide rows are read in 16-byte slices, 32 samples' slices in
// flight per step of the sequential sum (consecutive positions share their
// destination row).
__device__ __forceinline__ float batch_mean_grad(const float* g, const float* a, int32_t B) {
  float total = g[0] * a[0];
  int b = 1;
  if ((B & 3) == 0) {
    for (; b < 4; ++b) total = total + g[b] * a[b];
    for (; b + 32 <= B; b += 32) {
      float4 gv[8], av[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        gv[k] = *reinterpret_cast<const float4*>(g + b + 4 * k);
        av[k] = *reinterpret_cast<const float4*>(a + b + 4 * k);
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        total = total + gv[k].x * av[k].x;
        total = total + gv[k].y * av[k].y;
        total = total + gv[k].z * av[k].z;
        total = total + gv[k].w * av[k].w;
      }
    }
    for (; b + 4 <= B; b += 4) {
      const float4 gv = *reinterpret_cast<const float4*>(g + b);
      const float4 av = *reinterpret_cast<const float4*>(a + b);
      total = total + gv.x * av.x;
      total = total + gv.y * av.y;
      total = total + gv.z * av.z;
      total = total + gv.w * av.w;
    }
  } else {
    for (; b + 8 <= B; b += 8) {
      float gv[8], av[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        gv[k] = g[b + k];
        av[k] = a[b + k];
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) total = total + gv[k] * av[k];
    }
  }
  for (; b < B; ++b) total = total + g[b] * a[b];
  return total / static_cast<float>(B);
}

template <int RULE, bool UNI_T>
__global__ __launch_bounds__(kBatchBlock) void k_update_batch(plx_update_desc d, int32_t B) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kBatchBlock + threadIdx.x;
  if (e >= d.n) return;
  const bool live = d.dead ? d.dead[e] == 0 : e < d.live_end;
  if (!live) return;  // dead rows keep their values
  float den1 = 1.0f, den2 = 1.0f;
  if (RULE == PLX_RULE_ADAM && UNI_T) {
    const float step = d.step_t + 1.0f;
    den1 = 1.0f - adam_pow(d, d.p[1], step, 0);
    den2 = 1.0f - adam_pow(d, d.p[2], step, 1);
  }
  const float grad = batch_mean_grad(d.gfield + static_cast<int64_t>(d.dst[e]) * B,
                                     d.act + static_cast<int64_t>(d.src[e]) * B, B);
  constexpr int nstate =
      RULE == PLX_RULE_SGD ? 0 : (RULE == PLX_RULE_ADAM ? (UNI_T ? 2 : 3) : 1);
  float w = d.weight[e];
  float s0 = nstate >= 1 ? d.s0[e] : 0.0f;
  float s1 = nstate >= 2 ? d.s1[e] : 0.0f;
  float s2 = nstate >= 3 ? d.s2[e] : 0.0f;
  update_edge<RULE, UNI_T>(d, grad, den1, den2, w, s0, s1, s2);
  d.weight[e] = w;
  if (nstate >= 1) d.s0[e] = s0;
  if (nstate >= 2) d.s1[e] = s1;
  if (nstate >= 3) d.s2[e] = s2;
}

// The batch-mean update over tiles of <= 64 destination x 64 source units:
// the tile's gfield and act rows are staged in LDS 64 samples at a time
// (rows padded to 65 floats: lanes reading different rows at one sample hit
// different banks), and each edge (up to kTileEdges / kBatchBlock per lane)
// carries its running sum over the chunks, in sample order.
#ifndef PLX_BATCH_TILE_ROWS
#define PLX_BATCH_TILE_ROWS 64
#endif
constexpr int kTileRows = PLX_BATCH_TILE_ROWS;
static_assert(kTileRows > 0 && kTileRows <= 256 && (kTileRows & (kTileRows - 1)) == 0,
              "batched-update tile rows: a power of two that fits loc's 8-bit fields");
constexpr int kTileChunk = 64;
constexpr int kTileStride = kTileChunk + 4;  // 16-byte aligned rows, offset by 4 banks each
constexpr int kTileEdgesPer = 4;
constexpr int kTileEdges = kTileEdgesPer * kBatchBlock;

template <int RULE, bool UNI_T>
__global__ __launch_bounds__(kBatchBlock) void k_update_batch_tiles(plx_update_desc d, plx_batch_tiles t,
                                                                    int32_t B) {
  __shared__ __align__(16) float gs[kTileRows * kTileStride];
  __shared__ __align__(16) float as[kTileRows * kTileStride];
  const int k = blockIdx.x;
  const int j0 = t.tile_off[k], j1 = t.tile_off[k + 1];
  const int dbase = t.tile_base[2 * k], sbase = t.tile_base[2 * k + 1];
  int64_t pe[kTileEdgesPer];
  int ld[kTileEdgesPer], ls[kTileEdgesPer];
  bool use[kTileEdgesPer];
  float total[kTileEdgesPer];
#pragma unroll
  for (int i = 0; i < kTileEdgesPer; ++i) {
    const int j = j0 + static_cast<int>(threadIdx.x) + i * kBatchBlock;
    use[i] = j < j1;
    pe[i] = 0;
    ld[i] = ls[i] = 0;
    total[i] = 0.0f;
    if (use[i]) {
      pe[i] = t.pos[j];
      const uint32_t l = t.loc[j];
      // (masked to the tile: an entry outside it cannot reach past the LDS rows)
      ld[i] = static_cast<int>(l & 0xFFu) & (kTileRows - 1);
      ls[i] = static_cast<int>(l >> 8) & (kTileRows - 1);
      use[i] = d.dead ? d.dead[pe[i]] == 0 : pe[i] < d.live_end;
    }
  }
  // Rows [base, base + 64) x samples [c0, c0 + 64) of both fields (rows
  // past the last unit and samples past B are not read) go to registers, every
  // load issued before any is used; the next chunk's loads are in flight while
  // this chunk is summed from LDS.
  constexpr int kStage = kTileRows * kTileChunk / kBatchBlock;
  float vg[kStage], va[kStage];
  auto stage_load = [&](int c0) {
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
      const int q = static_cast<int>(threadIdx.x) + i * kBatchBlock;
      const int r = q / kTileChunk, c = q % kTileChunk;
      const bool inc = c0 + c < B;
      vg[i] = inc && dbase + r < t.num_units ? d.gfield[static_cast<int64_t>(dbase + r) * B + c0 + c] : 0.0f;
      va[i] = inc && sbase + r < t.num_units ? d.act[static_cast<int64_t>(sbase + r) * B + c0 + c] : 0.0f;
    }
  };
  stage_load(0);
  for (int c0 = 0; c0 < B; c0 += kTileChunk) {
    const int cn = min(kTileChunk, B - c0);
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
      const int q = static_cast<int>(threadIdx.x) + i * kBatchBlock;
      const int r = q / kTileChunk, c = q % kTileChunk;
      gs[r * kTileStride + c] = vg[i];
      as[r * kTileStride + c] = va[i];
    }
    __syncthreads();
    if (c0 + kTileChunk < B) stage_load(c0 + kTileChunk);
#pragma unroll
    for (int i = 0; i < kTileEdgesPer; ++i) {
      if (!use[i]) continue;
      const float* g = gs + ld[i] * kTileStride;
      const float* a = as + ls[i] * kTileStride;
      float s = total[i];
      int c = 0;
      if (c0 == 0) {
        s = g[0] * a[0];  // the sum starts from sample 0's term, not from +0.0
        c = 1;
      }
      // Up to the next multiple of 4 one sample at a time, then eight
      // samples per step from 16-byte LDS reads.
      for (; c < cn && (c & 3); ++c) s = s + g[c] * a[c];
      for (; c + 8 <= cn; c += 8) {
        const float4 x0 = *reinterpret_cast<const float4*>(g + c);
        const float4 x1 = *reinterpret_cast<const float4*>(g + c + 4);
        const float4 y0 = *reinterpret_cast<const float4*>(a + c);
        const float4 y1 = *reinterpret_cast<const float4*>(a + c + 4);
        s = s + x0.x * y0.x;
        s = s + x0.y * y0.y;
        s = s + x0.z * y0.z;
        s = s + x0.w * y0.w;
        s = s + x1.x * y1.x;
        s = s + x1.y * y1.y;
        s = s + x1.z * y1.z;
        s = s + x1.w * y1.w;
      }
      for (; c < cn; ++c) s = s + g[c] * a[c];
      total[i] = s;
    }
    __syncthreads();
  }
  float den1 = 1.0f, den2 = 1.0f;
  if (RULE == PLX_RULE_ADAM && UNI_T) {
    const float step = d.step_t + 1.0f;
    den1 = 1.0f - adam_pow(d, d.p[1], step, 0);
    den2 = 1.0f - adam_pow(d, d.p[2], step, 1);
  }
  constexpr int nstate =
      RULE == PLX_RULE_SGD ? 0 : (RULE == PLX_RULE_ADAM ? (UNI_T ? 2 : 3) : 1);
#pragma unroll
  for (int i = 0; i < kTileEdgesPer; ++i) {
    if (!use[i]) continue;
    const int64_t e = pe[i];
    const float grad = total[i] / static_cast<float>(B);
    float w = d.weight[e];
    float s0 = nstate >= 1 ? d.s0[e] : 0.0f;
    float s1 = nstate >= 2 ? d.s1[e] : 0.0f;
    float s2 = nstate >= 3 ? d.s2[e] : 0.0f;
    update_edge<RULE, UNI_T>(d, grad, den1, den2, w, s0, s1, s2);
    d.weight[e] = w;
    if (nstate >= 1) d.s0[e] = s0;
    if (nstate >= 2) d.s1[e] = s1;
    if (nstate >= 3) d.s2[e] = s2;
  }
}

template <typename T>
__global__ void k_reduce_batch(int64_t n, int32_t B, int32_t mode, const T* src, T* dst) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (u >= n) return;
  const T* x = src + u * B;
  T s = x[0];
  if (mode != PLX_REDUCE_FIRST) {
    // Eight samples' loads in flight per step of the sequential sum.
    int b = 1;
    for (; b + 8 <= B; b += 8) {
      T v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = x[b + k];
#pragma unroll
      for (int k = 0; k < 8; ++k) s = s + v[k];
    }
    for (; b < B; ++b) s = s + x[b];
  }
  if (mode == PLX_REDUCE_MEAN) s = s / static_cast<T>(B);
  dst[u] = s;
}

template <>
__global__ void k_reduce_batch<uint8_t>(int64_t n, int32_t B, int32_t mode, const uint8_t* src,
                                        uint8_t* dst) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (u < n) dst[u] = src[u * B];  // FIRST (the entry point refuses the rest)
}

// int32 sums wrap (two's complement), as numpy's and XLA's do.
template <>
__global__ void k_reduce_batch<int32_t>(int64_t n, int32_t B, int32_t mode, const int32_t* src,
                                        int32_t* dst) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (u >= n) return;
  const int32_t* x = src + u * B;
  uint32_t s = static_cast<uint32_t>(x[0]);
  if (mode == PLX_REDUCE_SUM)
    for (int b = 1; b < B; ++b) s += static_cast<uint32_t>(x[b]);
  dst[u] = static_cast<int32_t>(s);
}

__global__ void k_batch_mean(int32_t B, const float* losses, float* out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  float s = 0.0f;
  for (int b = 0; b < B; ++b) s = s + losses[b];
  *out = s / static_cast<float>(B);
}

// ---------------------------------------------------------------------------
// Small kernels: scatter, fill, losses, Philox, math probes.
// ---------------------------------------------------------------------------
__global__ void k_scatter(int32_t n, const int32_t* ids, const float* values, float* dst) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < n) dst[ids[k]] = values[k];
}

__global__ void k_fill(int64_t n, float value, float* dst) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (k < n) dst[k] = value;
}

constexpr int kPiece = 256;

// One 256-output piece per workgroup: each thread runs the loss program for
// one output (out slot 0, the seed, lands at the output's unit id; slot 1 is
// the loss term), then one lane folds the piece's terms in order from +0.0.
// Batched (B > 1): sample b = blockIdx.y reads and writes unit u at u * B + b,
// its targets at targets[b * n_out ..] and its piece sums at b * gridDim.x.
__global__ __launch_bounds__(kPiece) void k_loss_pieces(int32_t n_out, const int32_t* ids,
                                                       const float* targets, plx_program P,
                                                       float* piece_sums, int32_t B) {
  __shared__ float terms[kPiece];
  const int b = blockIdx.y;
  const int k = blockIdx.x * kPiece + threadIdx.x;
  if (k < n_out) {
    const int64_t u = static_cast<int64_t>(ids[k]) * B + b;
    terms[threadIdx.x] =
        run_program(P, u, load_loss_fields(P, u, b), 0.0f, targets[static_cast<int64_t>(b) * n_out + k], true);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int len = min(kPiece, n_out - static_cast<int>(blockIdx.x) * kPiece);
    float s = 0.0f;
    for (int j = 0; j < len; ++j) s = s + terms[j];
    piece_sums[static_cast<int64_t>(b) * gridDim.x + blockIdx.x] = s;
  }
}

// Folds n piece sums in order from +0.0 into *out, staging them through LDS
// (workgroup b: sums[b * n ..] into out[b]).
__global__ __launch_bounds__(1024) void k_fold_sums(int32_t n, const float* sums, float* out) {
  __shared__ float buf[1024];
  sums += static_cast<int64_t>(blockIdx.x) * n;
  out += blockIdx.x;
  float s = 0.0f;
  for (int base = 0; base < n; base += 1024) {
    const int len = min(1024, n - base);
    if (static_cast<int>(threadIdx.x) < len) buf[threadIdx.x] = sums[base + threadIdx.x];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int j = 0; j < len; ++j) s = s + buf[j];
    __syncthreads();
  }
  if (threadIdx.x == 0) *out = 0.0f + s;
}

constexpr int kSoftmaxMaxPieces = 1024;

// Workgroup b is sample b: unit u at u * B + b, targets[b * n ..], loss_out[b].
__global__ __launch_bounds__(1024) void k_softmax_ce(int32_t n, const int32_t* ids,
                                                     const float* act_base, const float* targets,
                                                     float* seed_base, float* loss_out, int32_t B) {
  __shared__ float red[1024];
  __shared__ float piece[kSoftmaxMaxPieces];
  __shared__ float bcast[2];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  targets += static_cast<int64_t>(b) * n;
  loss_out += b;
  auto at = [&](int k) { return static_cast<int64_t>(ids[k]) * B + b; };
  const float* act = act_base;
  float* seed_field = seed_base;
  // 1. max by a '>' scan from -inf (NaN is never taken), then a tree.
  float m = -__builtin_huge_valf();
  for (int k = tid; k < n; k += blockDim.x) {
    const float a = act[at(k)];
    if (a > m) m = a;
  }
  red[tid] = m;
  __syncthreads();
  for (int w = blockDim.x / 2; w > 0; w >>= 1) {
    if (tid < w && red[tid + w] > red[tid]) red[tid] = red[tid + w];
    __syncthreads();
  }
  const float peak = red[0];
  const int npieces = (n + kPiece - 1) / kPiece;
  // 2. sum of exp(a - peak), piecewise.
  for (int p = tid; p < npieces; p += blockDim.x) {
    float s = 0.0f;
    const int end = min(n, (p + 1) * kPiece);
    for (int k = p * kPiece; k < end; ++k) s = s + px::expf_(act[at(k)] - peak);
    piece[p] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float s = 0.0f;
    for (int p = 0; p < npieces; ++p) s = s + piece[p];
    bcast[0] = s;
    bcast[1] = px::logf_(s);
  }
  __syncthreads();
  const float total = bcast[0], log_sum = bcast[1];
  // 3. seeds and the piecewise loss fold.
  for (int p = tid; p < npieces; p += blockDim.x) {
    float s = 0.0f;
    const int end = min(n, (p + 1) * kPiece);
    for (int k = p * kPiece; k < end; ++k) {
      const float z = act[at(k)] - peak;
      const float t = targets[k];
      seed_field[at(k)] = px::expf_(z) / total - t;
      s = s + t * (log_sum - z);
    }
    piece[p] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float s = 0.0f;
    for (int p = 0; p < npieces; ++p) s = s + piece[p];
    *loss_out = 0.0f + s;
  }
}


__global__ void k_philox(int64_t n, const uint64_t* seeds, const uint64_t* ctrs, uint32_t* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = px::philox32(seeds[i], ctrs[i]);
}

__global__ void k_math(int32_t op, int64_t n, const float* x, const float* y, float* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  float r;
  switch (op) {
    case 0: r = px::expf_(v); break;
    case 1: r = px::logf_(v); break;
    case 2: r = px::tanhf_(v); break;
    case 3: r = px::sigmoidf_(v); break;
    case 4: r = sqrtf(v); break;
    case 6: r = px::cosf_(v); break;
    case 7: r = px::sinf_(v); break;
    case 8: r = px::log1pf_(v); break;
    case 9: r = px::expm1f_(v); break;
    default: r = px::pow_step(v, y[i]); break;
  }
  out[i] = r;
}

inline unsigned grid_for(int64_t n, int block) {
  return static_cast<unsigned>((n + block - 1) / block);
}

// The current device's CU count (queried once per device; 256 on MI355X).
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// A program's sizes are in range; fields read at a fixed unit only where
// the kernel honours them (the loss) and only among the program's fields.
bool program_ok(const plx_program& p, bool fixed_ok = false) {
  if (p.ninstr < 0 || p.ninstr > PLX_MAX_INSTR || p.nout < 0 || p.nout > PLX_MAX_OUTS) return false;
  if (p.nfields < 0 || p.nfields > PLX_MAX_FIELDS) return false;
  if (p.fixed_mask == 0) return true;
  return fixed_ok && (static_cast<uint32_t>(p.fixed_mask) >> p.nfields) == 0u;
}

template <int RULE, int M, bool FOLD, bool SAME_G, bool UNI_T, bool FAST>
void launch_tile_k(const plx_tile_desc& d, size_t lds, hipStream_t s) {
  // LDS beyond 64 KiB needs an explicit per-kernel opt-in.
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&k_tile<RULE, M, FOLD, SAME_G, UNI_T, FAST>),
      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  (void)attr;
  // One workgroup per superblock of tiles.
  k_tile<RULE, M, FOLD, SAME_G, UNI_T, FAST>
      <<<static_cast<unsigned>(d.nsuper), kTileBlock, lds, s>>>(d);
}
template <int RULE, int M, bool FOLD, bool SAME_G, bool UNI_T>
void launch_tile_g(const plx_tile_desc& d, size_t lds, hipStream_t s) {
  if (d.dst8 && !d.dead)
    launch_tile_k<RULE, M, FOLD, SAME_G, UNI_T, true>(d, lds, s);
  else
    launch_tile_k<RULE, M, FOLD, SAME_G, UNI_T, false>(d, lds, s);
}
// Instantiates only the meaningful variants: SAME_G needs a fold and an
// update, UNI_T is Adam's.
template <int RULE, int M, bool FOLD>
void launch_tile(const plx_tile_desc& d, size_t lds, hipStream_t s) {
  constexpr bool kSame = FOLD && RULE >= 0;
  const bool same = kSame && d.g == d.gfield;
  if constexpr (RULE == PLX_RULE_ADAM) {
    if (d.step_mode == 1) {
      if constexpr (kSame) {
        if (same) return launch_tile_g<RULE, M, FOLD, kSame, true>(d, lds, s);
      }
      return launch_tile_g<RULE, M, FOLD, false, true>(d, lds, s);
    }
  }
  if constexpr (kSame) {
    if (same) return launch_tile_g<RULE, M, FOLD, kSame, false>(d, lds, s);
  }
  launch_tile_g<RULE, M, FOLD, false, false>(d, lds, s);
}
template <int M, bool FOLD>
int dispatch_rule(const plx_tile_desc& d, size_t lds, hipStream_t s) {
  switch (d.update ? d.rule : -1) {
    case -1:
      // (no update: only a fold launches; the caller returns before otherwise)
      if constexpr (FOLD) launch_tile<-1, M, FOLD>(d, lds, s);
      break;
    case PLX_RULE_SGD: launch_tile<PLX_RULE_SGD, M, FOLD>(d, lds, s); break;
    case PLX_RULE_MOMENTUM: launch_tile<PLX_RULE_MOMENTUM, M, FOLD>(d, lds, s); break;
    case PLX_RULE_ADAM: launch_tile<PLX_RULE_ADAM, M, FOLD>(d, lds, s); break;
    case PLX_RULE_RMSPROP: launch_tile<PLX_RULE_RMSPROP, M, FOLD>(d, lds, s); break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_backward_tiles: unknown rule");
  }
  return PLX_OK;
}

}  // namespace

int plx_detail::forward_launch_shape(const plx_forward_desc* d, const char* who, unsigned* grid,
                                     unsigned* block) {
  const std::string w(who);
  *grid = 0;
  *block = kFwdBlock;
  if (!d) return fail(PLX_ERR_INVALID, (w + ": null descriptor").c_str());
  if (d->nrows < 0) return fail(PLX_ERR_INVALID, (w + ": negative nrows").c_str());
  if (d->nrows == 0) return PLX_OK;
  if (!d->row_unit || !d->row_ptr || !d->src || !d->weight || !d->x)
    return fail(PLX_ERR_INVALID, (w + ": null column").c_str());
  if (!program_ok(d->apply)) return fail(PLX_ERR_INVALID, (w + ": bad program").c_str());
  if (d->tbl_len < 0 || d->tbl_len > PLX_MAX_TBL)
    return fail(PLX_ERR_INVALID, (w + ": tbl_len must be in [0, PLX_MAX_TBL]").c_str());
  if (!d->fin.level || !d->fin.is_input)
    return fail(PLX_ERR_INVALID, (w + ": fin.level and fin.is_input are required").c_str());
  if (d->prune_prog && (!d->prune_sink || d->num_units <= 0))
    return fail(PLX_ERR_INVALID, (w + ": prune_prog needs prune_sink and num_units").c_str());
  const unsigned nblk = grid_for(d->nrows, kFwdRows);
  const unsigned cap = static_cast<unsigned>(cu_count() * kFwdPerCU);
  *grid = nblk < cap ? nblk : cap;
  return PLX_OK;
}

extern "C" {

const char* plx_last_error(void) { return plx_detail::g_last_error.c_str(); }

int32_t plx_abi_version(void) { return 28; }

int plx_struct_sizes(int64_t* out, int32_t n) {
  const int64_t sizes[20] = {
      sizeof(plx_program),          sizeof(plx_finalize),
      sizeof(plx_forward_desc),     sizeof(plx_tile_desc),
      sizeof(plx_partials_desc),    sizeof(plx_update_desc),
      sizeof(plx_site_prog),        sizeof(plx_site_desc),
      sizeof(plx_sort_key),         sizeof(plx_sort_desc),
      sizeof(plx_grow_filter_desc), sizeof(plx_grow_col),
      sizeof(plx_grow_claim_desc),  sizeof(plx_unit_col),
      sizeof(plx_bwd_batch_desc),   sizeof(plx_batch_tiles),
      sizeof(plx_tile_build_desc),  sizeof(plx_gen_fold_desc),
      sizeof(plx_merge_desc),       sizeof(plx_merge_gather_desc)};
  for (int32_t k = 0; k < n && k < 20; ++k) out[k] = sizes[k];
  return 20;
}

int plx_forward_bucket(const plx_forward_desc* d, void* stream) {
  unsigned grid = 0, block = 0;
  const int rc = plx_detail::forward_launch_shape(d, "plx_forward_bucket", &grid, &block);
  if (rc || grid == 0) return rc;
  const bool prune = d->prune_prog != nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (d->monoid) {
    case PLX_MONOID_SUM:
      if (prune)
        k_forward<PLX_MONOID_SUM, true><<<grid, kFwdBlock, 0, s>>>(*d);
      else
        k_forward<PLX_MONOID_SUM, false><<<grid, kFwdBlock, 0, s>>>(*d);
      break;
    case PLX_MONOID_PROD:
      if (prune)
        k_forward<PLX_MONOID_PROD, true><<<grid, kFwdBlock, 0, s>>>(*d);
      else
        k_forward<PLX_MONOID_PROD, false><<<grid, kFwdBlock, 0, s>>>(*d);
      break;
    case PLX_MONOID_MAX:
      if (prune)
        k_forward<PLX_MONOID_MAX, true><<<grid, kFwdBlock, 0, s>>>(*d);
      else
        k_forward<PLX_MONOID_MAX, false><<<grid, kFwdBlock, 0, s>>>(*d);
      break;
    case PLX_MONOID_MIN:
      if (prune)
        k_forward<PLX_MONOID_MIN, true><<<grid, kFwdBlock, 0, s>>>(*d);
      else
        k_forward<PLX_MONOID_MIN, false><<<grid, kFwdBlock, 0, s>>>(*d);
      break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_forward_bucket: unknown monoid");
  }
  return check_launch("plx_forward_bucket");
}

int plx_backward_tiles(const plx_tile_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_backward_tiles: null descriptor");
  if (d->ntiles < 0 || d->tile_size <= 0 || d->tile_size % 4 ||
      d->tile_size > 4 * kTileQuads * kTileBlock)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: tile_size must be a positive multiple of 4 <= 4096");
  if (d->base % 4 || d->end % 4 || d->end < d->base)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: base/end must be multiples of 4");
  if (d->ntiles == 0 || d->end == d->base) return PLX_OK;
  if (d->nsuper <= 0 || d->nsuper > d->ntiles || !d->tile_pos || !d->super_tile)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: tile / superblock tables missing");
  if (!d->src || !d->dst || !d->weight)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: null column");
  if (d->dst8 && !d->blk_dst0) return fail(PLX_ERR_INVALID, "plx_backward_tiles: dst8 needs blk_dst0");
  if (d->step_mode != 0 && d->step_mode != 1)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: step_mode must be 0 or 1");
  if (d->fold && (!d->tile_info || !d->grp_off || !d->grp || !d->sorted_rank || !d->g || !d->cold_partial ||
                  (d->nhot > 0 && !d->hot_sb)))
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: fold metadata missing");
  if (d->update && (!d->gfield || !d->act))
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: update fields missing");
  if (d->update && (d->rule == PLX_RULE_MOMENTUM || d->rule == PLX_RULE_RMSPROP) && !d->s0)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: state column missing");
  if (d->update && d->rule == PLX_RULE_ADAM &&
      (!d->s0 || !d->s1 || (d->step_mode == 0 && !d->s2)))
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: Adam state columns missing");
  if (!d->fold && !d->update) return PLX_OK;
  if (d->fold && (d->nhot < 0 || d->nhot > 32767))
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: nhot must be in [0, 32767]");
  if (d->tbl_len < 0 || d->tbl_len > PLX_MAX_TBL)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: tbl_len must be in [0, PLX_MAX_TBL]");
  const size_t tbl = d->update ? static_cast<size_t>(d->tbl_len) * 4 : 0;
  const size_t lds = (d->fold ? static_cast<size_t>(d->tile_size) * 4 +
                                    static_cast<size_t>((2 * d->tile_size + 15) & ~15) + kTileInfo * 4 +
                                    static_cast<size_t>((d->nhot + 3) & ~3) * 4
                              : 0) + tbl;
  if (lds > 160 * 1024) return fail(PLX_ERR_UNSUPPORTED, "plx_backward_tiles: tile does not fit in LDS");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = PLX_OK;
  if (!d->fold) {
    rc = dispatch_rule<PLX_MONOID_SUM, false>(*d, lds, s);
  } else {
    switch (d->monoid) {
      case PLX_MONOID_SUM: rc = dispatch_rule<PLX_MONOID_SUM, true>(*d, lds, s); break;
      case PLX_MONOID_PROD: rc = dispatch_rule<PLX_MONOID_PROD, true>(*d, lds, s); break;
      case PLX_MONOID_MAX: rc = dispatch_rule<PLX_MONOID_MAX, true>(*d, lds, s); break;
      case PLX_MONOID_MIN: rc = dispatch_rule<PLX_MONOID_MIN, true>(*d, lds, s); break;
      default: return fail(PLX_ERR_UNSUPPORTED, "plx_backward_tiles: unknown monoid");
    }
  }
  if (rc) return rc;
  return check_launch("plx_backward_tiles");
}

int plx_backward_partials(const plx_partials_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_backward_partials: null descriptor");
  if (d->nrows < 0) return fail(PLX_ERR_INVALID, "plx_backward_partials: negative nrows");
  if (d->nrows == 0) return PLX_OK;
  if (!d->row_unit) return fail(PLX_ERR_INVALID, "plx_backward_partials: null row_unit");
  if (d->nparts < 0 || (d->nparts > 0 && !d->part_rows))
    return fail(PLX_ERR_INVALID, "plx_backward_partials: part_rows missing");
  if (d->row_hot && (d->nhot < 0 || d->nsuper < 0 || (d->nhot > 0 && !d->hot_sb)))
    return fail(PLX_ERR_INVALID, "plx_backward_partials: hot partials missing");
  if (d->row_cold && (!d->cold_partial || !d->cold_sb || !d->cold_idx))
    return fail(PLX_ERR_INVALID, "plx_backward_partials: cold partials missing");
  if (!program_ok(d->apply)) return fail(PLX_ERR_INVALID, "plx_backward_partials: bad program");
  if (!d->fin.level || !d->fin.is_input)
    return fail(PLX_ERR_INVALID, "plx_backward_partials: fin.level and fin.is_input are required");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nhot_rows = d->row_hot ? d->nhot : 0;
  if (nhot_rows > d->nrows) return fail(PLX_ERR_INVALID, "plx_backward_partials: nhot > nrows");
  const int hot_wgs = nhot_rows > 0 && d->nsuper > 0 ? static_cast<int>(grid_for(nhot_rows, kHotCols)) : 0;
  const int cold_wgs = d->nparts > 0 ? d->nparts : 0;
  if (hot_wgs + cold_wgs == 0) return PLX_OK;
  const unsigned grid = static_cast<unsigned>(hot_wgs + cold_wgs);
  switch (d->monoid) {
    case PLX_MONOID_SUM: k_finalize<PLX_MONOID_SUM><<<grid, kFinBlock, 0, s>>>(*d, hot_wgs); break;
    case PLX_MONOID_PROD: k_finalize<PLX_MONOID_PROD><<<grid, kFinBlock, 0, s>>>(*d, hot_wgs); break;
    case PLX_MONOID_MAX: k_finalize<PLX_MONOID_MAX><<<grid, kFinBlock, 0, s>>>(*d, hot_wgs); break;
    case PLX_MONOID_MIN: k_finalize<PLX_MONOID_MIN><<<grid, kFinBlock, 0, s>>>(*d, hot_wgs); break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_backward_partials: unknown monoid");
  }
  return check_launch("plx_backward_partials");
}

int plx_update_conn(const plx_update_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_update_conn: null descriptor");
  if (d->n < 0) return fail(PLX_ERR_INVALID, "plx_update_conn: negative n");
  if (d->n == 0) return PLX_OK;
  if (d->n % 4 != 0) return fail(PLX_ERR_INVALID, "plx_update_conn: n must be a multiple of 4");
  if (!d->src || !d->dst || !d->weight || !d->gfield || !d->act)
    return fail(PLX_ERR_INVALID, "plx_update_conn: null column");
  if (d->step_mode != 0 && d->step_mode != 1)
    return fail(PLX_ERR_INVALID, "plx_update_conn: step_mode must be 0 or 1");
  if ((d->rule == PLX_RULE_MOMENTUM || d->rule == PLX_RULE_RMSPROP) && !d->s0)
    return fail(PLX_ERR_INVALID, "plx_update_conn: state column missing");
  if (d->rule == PLX_RULE_ADAM && (!d->s0 || !d->s1 || (d->step_mode == 0 && !d->s2)))
    return fail(PLX_ERR_INVALID, "plx_update_conn: Adam state columns missing");
  if (d->tbl_len < 0 || d->tbl_len > PLX_MAX_TBL)
    return fail(PLX_ERR_INVALID, "plx_update_conn: tbl_len must be in [0, PLX_MAX_TBL]");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Four workgroups per CU stride over the positions.
  const unsigned quads_grid = grid_for(d->n / 4, kUpdBlock);
  const unsigned grid = quads_grid < 1024u ? quads_grid : 1024u;
  switch (d->rule) {
    case PLX_RULE_SGD: k_update<PLX_RULE_SGD, false><<<grid, kUpdBlock, 0, s>>>(*d); break;
    case PLX_RULE_MOMENTUM: k_update<PLX_RULE_MOMENTUM, false><<<grid, kUpdBlock, 0, s>>>(*d); break;
    case PLX_RULE_ADAM:
      if (d->step_mode == 1)
        k_update<PLX_RULE_ADAM, true><<<grid, kUpdBlock, 0, s>>>(*d);
      else
        k_update<PLX_RULE_ADAM, false><<<grid, kUpdBlock, 0, s>>>(*d);
      break;
    case PLX_RULE_RMSPROP: k_update<PLX_RULE_RMSPROP, false><<<grid, kUpdBlock, 0, s>>>(*d); break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_update_conn: unknown rule");
  }
  return check_launch("plx_update_conn");
}

int plx_scatter_f32(int32_t n, const int32_t* ids, const float* values, float* dst,
                    void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_scatter_f32: negative n");
  if (n == 0) return PLX_OK;
  if (!ids || !values || !dst) return fail(PLX_ERR_INVALID, "plx_scatter_f32: null pointer");
  k_scatter<<<grid_for(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(n, ids, values, dst);
  return check_launch("plx_scatter_f32");
}

int plx_fill_f32(int64_t n, float value, float* dst, void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_fill_f32: negative n");
  if (n == 0) return PLX_OK;
  if (!dst) return fail(PLX_ERR_INVALID, "plx_fill_f32: null pointer");
  k_fill<<<grid_for(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(n, value, dst);
  return check_launch("plx_fill_f32");
}

int plx_loss_elementwise(int32_t n_out, const int32_t* output_ids, const float* targets,
                         const plx_program* term, float* seed_field, float* partials,
                         float* loss_out, void* stream) {
  if (n_out < 0) return fail(PLX_ERR_INVALID, "plx_loss_elementwise: negative n_out");
  if (!term || !loss_out || !partials)
    return fail(PLX_ERR_INVALID, "plx_loss_elementwise: null pointer");
  if (!program_ok(*term, true)) return fail(PLX_ERR_INVALID, "plx_loss_elementwise: bad program");
  if (n_out > 0 && (!output_ids || !targets || !seed_field))
    return fail(PLX_ERR_INVALID, "plx_loss_elementwise: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  plx_program p = *term;
  p.outs[0] = seed_field;  // slot 0: the seed, stored at the output unit
  p.outs[1] = nullptr;     // slot 1: the term, returned to the kernel
  if (p.nout < 2) p.nout = 2;
  const int npieces = (n_out + kPiece - 1) / kPiece;
  if (npieces > 0) {
    k_loss_pieces<<<npieces, kPiece, 0, s>>>(n_out, output_ids, targets, p, partials, 1);
    int rc = check_launch("plx_loss_elementwise");
    if (rc) return rc;
  }
  k_fold_sums<<<1, 1024, 0, s>>>(npieces, partials, loss_out);
  return check_launch("plx_loss_elementwise");
}

int plx_loss_softmax_ce(int32_t n_out, const int32_t* output_ids, const float* act,
                        const float* targets, float* seed_field, float* loss_out,
                        void* stream) {
  if (n_out < 0) return fail(PLX_ERR_INVALID, "plx_loss_softmax_ce: negative n_out");
  if (n_out > kSoftmaxMaxPieces * kPiece)
    return fail(PLX_ERR_UNSUPPORTED, "plx_loss_softmax_ce: more than 262144 outputs");
  if (!loss_out || (n_out > 0 && (!output_ids || !act || !targets || !seed_field)))
    return fail(PLX_ERR_INVALID, "plx_loss_softmax_ce: null pointer");
  k_softmax_ce<<<1, 1024, 0, static_cast<hipStream_t>(stream)>>>(n_out, output_ids, act,
                                                                  targets, seed_field, loss_out, 1);
  return check_launch("plx_loss_softmax_ce");
}

// ---- batched steps ---------------------------------------------------------
int plx_forward_batch(const plx_forward_desc* d, int32_t batch, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_forward_batch: null descriptor");
  if (batch < 1) return fail(PLX_ERR_INVALID, "plx_forward_batch: batch must be >= 1");
  if (d->nrows < 0) return fail(PLX_ERR_INVALID, "plx_forward_batch: negative nrows");
  if (d->nrows == 0) return PLX_OK;
  if (!d->row_unit || !d->row_ptr || !d->src || !d->weight || !d->x)
    return fail(PLX_ERR_INVALID, "plx_forward_batch: null column");
  if (!program_ok(d->apply)) return fail(PLX_ERR_INVALID, "plx_forward_batch: bad program");
  if (!d->fin.level || !d->fin.is_input)
    return fail(PLX_ERR_INVALID, "plx_forward_batch: fin.level and fin.is_input are required");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned block = batch >= kBatchBlock ? kBatchBlock : static_cast<unsigned>((batch + 63) / 64 * 64);
  const unsigned grid = static_cast<unsigned>(d->nrows);
  if (batch % 4 == 0 && batch >= 128 && d->nrows >= 256) {
    // 16-byte row loads: x rows are 16-byte aligned when B is a multiple of 4.
    // (A level of few rows keeps a 256-lane workgroup per row: with one wave
    // per row it would leave the GPU idle.)
    switch (d->monoid) {
      case PLX_MONOID_SUM: k_forward_batch4<PLX_MONOID_SUM><<<grid, 64, 0, s>>>(*d, batch); break;
      case PLX_MONOID_PROD: k_forward_batch4<PLX_MONOID_PROD><<<grid, 64, 0, s>>>(*d, batch); break;
      case PLX_MONOID_MAX: k_forward_batch4<PLX_MONOID_MAX><<<grid, 64, 0, s>>>(*d, batch); break;
      case PLX_MONOID_MIN: k_forward_batch4<PLX_MONOID_MIN><<<grid, 64, 0, s>>>(*d, batch); break;
      default: return fail(PLX_ERR_UNSUPPORTED, "plx_forward_batch: unknown monoid");
    }
    return check_launch("plx_forward_batch");
  }
  switch (d->monoid) {
    case PLX_MONOID_SUM: k_forward_batch<PLX_MONOID_SUM><<<grid, block, 0, s>>>(*d, batch); break;
    case PLX_MONOID_PROD: k_forward_batch<PLX_MONOID_PROD><<<grid, block, 0, s>>>(*d, batch); break;
    case PLX_MONOID_MAX: k_forward_batch<PLX_MONOID_MAX><<<grid, block, 0, s>>>(*d, batch); break;
    case PLX_MONOID_MIN: k_forward_batch<PLX_MONOID_MIN><<<grid, block, 0, s>>>(*d, batch); break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_forward_batch: unknown monoid");
  }
  return check_launch("plx_forward_batch");
}

int plx_backward_batch(const plx_bwd_batch_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_backward_batch: null descriptor");
  if (d->batch < 1) return fail(PLX_ERR_INVALID, "plx_backward_batch: batch must be >= 1");
  if (d->nrows < 0) return fail(PLX_ERR_INVALID, "plx_backward_batch: negative nrows");
  if (d->nrows == 0) return PLX_OK;
  if (!d->row_unit || !d->row_ptr || !d->dst || !d->weight || !d->g)
    return fail(PLX_ERR_INVALID, "plx_backward_batch: null column");
  if (!program_ok(d->apply)) return fail(PLX_ERR_INVALID, "plx_backward_batch: bad program");
  if (!d->fin.level || !d->fin.is_input)
    return fail(PLX_ERR_INVALID, "plx_backward_batch: fin.level and fin.is_input are required");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int batch = d->batch;
  const unsigned block = batch >= kBatchBlock ? kBatchBlock : static_cast<unsigned>((batch + 63) / 64 * 64);
  const unsigned grid = static_cast<unsigned>(d->nrows);
  if (batch % 4 == 0 && batch >= 128 && d->nrows >= 256) {
    // 16-byte row loads: g rows are 16-byte aligned when B is a multiple of 4
    // (few rows: the 256-lane form, as for the forward).
    switch (d->monoid) {
      case PLX_MONOID_SUM: k_backward_batch4<PLX_MONOID_SUM><<<grid, 64, 0, s>>>(*d); break;
      case PLX_MONOID_PROD: k_backward_batch4<PLX_MONOID_PROD><<<grid, 64, 0, s>>>(*d); break;
      case PLX_MONOID_MAX: k_backward_batch4<PLX_MONOID_MAX><<<grid, 64, 0, s>>>(*d); break;
      case PLX_MONOID_MIN: k_backward_batch4<PLX_MONOID_MIN><<<grid, 64, 0, s>>>(*d); break;
      default: return fail(PLX_ERR_UNSUPPORTED, "plx_backward_batch: unknown monoid");
    }
    return check_launch("plx_backward_batch");
  }
  switch (d->monoid) {
    case PLX_MONOID_SUM: k_backward_batch<PLX_MONOID_SUM><<<grid, block, 0, s>>>(*d); break;
    case PLX_MONOID_PROD: k_backward_batch<PLX_MONOID_PROD><<<grid, block, 0, s>>>(*d); break;
    case PLX_MONOID_MAX: k_backward_batch<PLX_MONOID_MAX><<<grid, block, 0, s>>>(*d); break;
    case PLX_MONOID_MIN: k_backward_batch<PLX_MONOID_MIN><<<grid, block, 0, s>>>(*d); break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_backward_batch: unknown monoid");
  }
  return check_launch("plx_backward_batch");
}

int plx_backward_lists(const plx_bwd_batch_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_backward_lists: null descriptor");
  if (d->batch != 1) return fail(PLX_ERR_INVALID, "plx_backward_lists: batch must be 1");
  if (d->nrows < 0) return fail(PLX_ERR_INVALID, "plx_backward_lists: negative nrows");
  if (d->nrows == 0) return PLX_OK;
  if (!d->row_unit || !d->row_ptr || !d->dst || !d->weight || !d->g)
    return fail(PLX_ERR_INVALID, "plx_backward_lists: null column");
  if (!program_ok(d->apply)) return fail(PLX_ERR_INVALID, "plx_backward_lists: bad program");
  if (!d->fin.level || !d->fin.is_input)
    return fail(PLX_ERR_INVALID, "plx_backward_lists: fin.level and fin.is_input are required");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(d->nrows, kBatchBlock);
  switch (d->monoid) {
    case PLX_MONOID_SUM: k_backward_lists<PLX_MONOID_SUM><<<grid, kBatchBlock, 0, s>>>(*d); break;
    case PLX_MONOID_PROD: k_backward_lists<PLX_MONOID_PROD><<<grid, kBatchBlock, 0, s>>>(*d); break;
    case PLX_MONOID_MAX: k_backward_lists<PLX_MONOID_MAX><<<grid, kBatchBlock, 0, s>>>(*d); break;
    case PLX_MONOID_MIN: k_backward_lists<PLX_MONOID_MIN><<<grid, kBatchBlock, 0, s>>>(*d); break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_backward_lists: unknown monoid");
  }
  return check_launch("plx_backward_lists");
}

int plx_gather_edges(int64_t n, const int32_t* pos, const float* weight, const uint8_t* dead,
                     float* out_weight, uint8_t* out_live, void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_gather_edges: negative n");
  if (n == 0) return PLX_OK;
  if (!pos || (out_weight && !weight)) return fail(PLX_ERR_INVALID, "plx_gather_edges: null pointer");
  k_gather_edges<<<grid_for(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(n, pos, weight, dead,
                                                                                  out_weight, out_live);
  return check_launch("plx_gather_edges");
}

int plx_update_batch(const plx_update_desc* d, int32_t batch, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_update_batch: null descriptor");
  if (batch < 1) return fail(PLX_ERR_INVALID, "plx_update_batch: batch must be >= 1");
  if (d->n < 0) return fail(PLX_ERR_INVALID, "plx_update_batch: negative n");
  if (d->n == 0) return PLX_OK;
  if (!d->src || !d->dst || !d->weight || !d->gfield || !d->act)
    return fail(PLX_ERR_INVALID, "plx_update_batch: null column");
  if (d->step_mode != 0 && d->step_mode != 1)
    return fail(PLX_ERR_INVALID, "plx_update_batch: step_mode must be 0 or 1");
  if ((d->rule == PLX_RULE_MOMENTUM || d->rule == PLX_RULE_RMSPROP) && !d->s0)
    return fail(PLX_ERR_INVALID, "plx_update_batch: state column missing");
  if (d->rule == PLX_RULE_ADAM && (!d->s0 || !d->s1 || (d->step_mode == 0 && !d->s2)))
    return fail(PLX_ERR_INVALID, "plx_update_batch: Adam state columns missing");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(d->n, kBatchBlock);
  switch (d->rule) {
    case PLX_RULE_SGD: k_update_batch<PLX_RULE_SGD, false><<<grid, kBatchBlock, 0, s>>>(*d, batch); break;
    case PLX_RULE_MOMENTUM:
      k_update_batch<PLX_RULE_MOMENTUM, false><<<grid, kBatchBlock, 0, s>>>(*d, batch);
      break;
    case PLX_RULE_ADAM:
      if (d->step_mode == 1)
        k_update_batch<PLX_RULE_ADAM, true><<<grid, kBatchBlock, 0, s>>>(*d, batch);
      else
        k_update_batch<PLX_RULE_ADAM, false><<<grid, kBatchBlock, 0, s>>>(*d, batch);
      break;
    case PLX_RULE_RMSPROP:
      k_update_batch<PLX_RULE_RMSPROP, false><<<grid, kBatchBlock, 0, s>>>(*d, batch);
      break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_update_batch: unknown rule");
  }
  return check_launch("plx_update_batch");
}

int plx_batch_tile_limits(int32_t* rows, int32_t* edges) {
  if (!rows || !edges) return fail(PLX_ERR_INVALID, "plx_batch_tile_limits: null pointer");
  *rows = kTileRows;
  *edges = kTileEdges;
  return PLX_OK;
}

int plx_update_batch_tiles(const plx_update_desc* d, const plx_batch_tiles* t, int32_t batch,
                           void* stream) {
  if (!d || !t) return fail(PLX_ERR_INVALID, "plx_update_batch_tiles: null descriptor");
  if (batch < 1) return fail(PLX_ERR_INVALID, "plx_update_batch_tiles: batch must be >= 1");
  if (t->ntiles < 0 || t->num_units < 0) return fail(PLX_ERR_INVALID, "plx_update_batch_tiles: negative size");
  if (t->ntiles == 0 || d->n == 0) return PLX_OK;
  if (!t->tile_off || !t->tile_base || !t->pos || !t->loc)
    return fail(PLX_ERR_INVALID, "plx_update_batch_tiles: null tile table");
  if (!d->weight || !d->gfield || !d->act) return fail(PLX_ERR_INVALID, "plx_update_batch_tiles: null column");
  if (d->step_mode != 0 && d->step_mode != 1)
    return fail(PLX_ERR_INVALID, "plx_update_batch_tiles: step_mode must be 0 or 1");
  if ((d->rule == PLX_RULE_MOMENTUM || d->rule == PLX_RULE_RMSPROP) && !d->s0)
    return fail(PLX_ERR_INVALID, "plx_update_batch_tiles: state column missing");
  if (d->rule == PLX_RULE_ADAM && (!d->s0 || !d->s1 || (d->step_mode == 0 && !d->s2)))
    return fail(PLX_ERR_INVALID, "plx_update_batch_tiles: Adam state columns missing");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>(t->ntiles);
  switch (d->rule) {
    case PLX_RULE_SGD: k_update_batch_tiles<PLX_RULE_SGD, false><<<grid, kBatchBlock, 0, s>>>(*d, *t, batch); break;
    case PLX_RULE_MOMENTUM:
      k_update_batch_tiles<PLX_RULE_MOMENTUM, false><<<grid, kBatchBlock, 0, s>>>(*d, *t, batch);
      break;
    case PLX_RULE_ADAM:
      if (d->step_mode == 1)
        k_update_batch_tiles<PLX_RULE_ADAM, true><<<grid, kBatchBlock, 0, s>>>(*d, *t, batch);
      else
        k_update_batch_tiles<PLX_RULE_ADAM, false><<<grid, kBatchBlock, 0, s>>>(*d, *t, batch);
      break;
    case PLX_RULE_RMSPROP:
      k_update_batch_tiles<PLX_RULE_RMSPROP, false><<<grid, kBatchBlock, 0, s>>>(*d, *t, batch);
      break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_update_batch_tiles: unknown rule");
  }
  return check_launch("plx_update_batch_tiles");
}

int plx_loss_elementwise_batch(int32_t n_out, const int32_t* output_ids, const float* targets,
                               const plx_program* term, float* seed_field, float* partials,
                               float* losses, int32_t batch, void* stream) {
  if (n_out < 0 || batch < 1) return fail(PLX_ERR_INVALID, "plx_loss_elementwise_batch: bad size");
  if (!term || !losses || !partials)
    return fail(PLX_ERR_INVALID, "plx_loss_elementwise_batch: null pointer");
  if (!program_ok(*term, true)) return fail(PLX_ERR_INVALID, "plx_loss_elementwise_batch: bad program");
  if (n_out > 0 && (!output_ids || !targets || !seed_field))
    return fail(PLX_ERR_INVALID, "plx_loss_elementwise_batch: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  plx_program p = *term;
  p.outs[0] = seed_field;
  p.outs[1] = nullptr;
  if (p.nout < 2) p.nout = 2;
  const int npieces = (n_out + kPiece - 1) / kPiece;
  if (npieces > 0) {
    k_loss_pieces<<<dim3(npieces, batch), kPiece, 0, s>>>(n_out, output_ids, targets, p, partials, batch);
    int rc = check_launch("plx_loss_elementwise_batch");
    if (rc) return rc;
  }
  k_fold_sums<<<batch, 1024, 0, s>>>(npieces, partials, losses);
  return check_launch("plx_loss_elementwise_batch");
}

int plx_loss_softmax_ce_batch(int32_t n_out, const int32_t* output_ids, const float* act,
                              const float* targets, float* seed_field, float* losses,
                              int32_t batch, void* stream) {
  if (n_out < 0 || batch < 1) return fail(PLX_ERR_INVALID, "plx_loss_softmax_ce_batch: bad size");
  if (n_out > kSoftmaxMaxPieces * kPiece)
    return fail(PLX_ERR_UNSUPPORTED, "plx_loss_softmax_ce_batch: more than 262144 outputs");
  if (!losses || (n_out > 0 && (!output_ids || !act || !targets || !seed_field)))
    return fail(PLX_ERR_INVALID, "plx_loss_softmax_ce_batch: null pointer");
  k_softmax_ce<<<batch, 1024, 0, static_cast<hipStream_t>(stream)>>>(n_out, output_ids, act, targets,
                                                                      seed_field, losses, batch);
  return check_launch("plx_loss_softmax_ce_batch");
}

int plx_batch_mean(int32_t batch, const float* losses, float* out, void* stream) {
  if (batch < 1 || !losses || !out) return fail(PLX_ERR_INVALID, "plx_batch_mean: bad argument");
  k_batch_mean<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(batch, losses, out);
  return check_launch("plx_batch_mean");
}

int plx_reduce_batch(int64_t n, int32_t batch, int32_t mode, int32_t kind, const void* src, void* dst,
                     void* stream) {
  if (n < 0 || batch < 1) return fail(PLX_ERR_INVALID, "plx_reduce_batch: bad size");
  if (mode < PLX_REDUCE_MEAN || mode > PLX_REDUCE_FIRST)
    return fail(PLX_ERR_INVALID, "plx_reduce_batch: unknown mode");
  if (kind == PLX_COL_I32 && mode == PLX_REDUCE_MEAN)
    return fail(PLX_ERR_INVALID, "plx_reduce_batch: MEAN needs a float32 column");
  if (kind == PLX_COL_U8 && mode != PLX_REDUCE_FIRST)
    return fail(PLX_ERR_INVALID, "plx_reduce_batch: a byte column reduces by FIRST only");
  if (n == 0) return PLX_OK;
  if (!src || !dst) return fail(PLX_ERR_INVALID, "plx_reduce_batch: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(n, 256);
  switch (kind) {
    case PLX_COL_F32:
      k_reduce_batch<float><<<grid, 256, 0, s>>>(n, batch, mode, static_cast<const float*>(src),
                                                static_cast<float*>(dst));
      break;
    case PLX_COL_I32:
      k_reduce_batch<int32_t><<<grid, 256, 0, s>>>(n, batch, mode, static_cast<const int32_t*>(src),
                                                  static_cast<int32_t*>(dst));
      break;
    case PLX_COL_U8:
      k_reduce_batch<uint8_t><<<grid, 256, 0, s>>>(n, batch, mode, static_cast<const uint8_t*>(src),
                                                  static_cast<uint8_t*>(dst));
      break;
    default: return fail(PLX_ERR_INVALID, "plx_reduce_batch: unknown column kind");
  }
  return check_launch("plx_reduce_batch");
}

int plx_philox32(int64_t n, const uint64_t* seeds, const uint64_t* ctrs, uint32_t* out,
                 void* stream) {
  if (n < 0) return fail(PLX_ERR_INVALID, "plx_philox32: negative n");
  if (n == 0) return PLX_OK;
  if (!seeds || !ctrs || !out) return fail(PLX_ERR_INVALID, "plx_philox32: null pointer");
  k_philox<<<grid_for(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(n, seeds, ctrs, out);
  return check_launch("plx_philox32");
}

int plx_eval_math(int32_t op, int64_t n, const float* x, const float* y, float* out,
                  void* stream) {
  if (n < 0 || op < 0 || op > 9) return fail(PLX_ERR_INVALID, "plx_eval_math: bad argument");
  if (n == 0) return PLX_OK;
  if (!x || !out || (op == 5 && !y)) return fail(PLX_ERR_INVALID, "plx_eval_math: null pointer");
  k_math<<<grid_for(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(op, n, x, y, out);
  return check_launch("plx_eval_math");
}

}  // extern "C"
