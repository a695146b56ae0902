// plastax_hip.hip -- gfx950 kernels of the streaming edge-arena step and the
// C ABI declared in include/plastax_hip.h.
//
// Data layout (built by plastax_amd/_layout.py): every bucket's edge columns
// live in one physical slab, destination-sorted inside each bucket (live edges
// ordered by (dst, logical slot), then the bucket's dead slots). The backward
// transpose reduce works on fixed tiles of that order: per-(tile, source)
// partials, folded per superblock of tiles, then across superblocks. All folds
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
#include "px_math.h"

namespace {

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

// ---------------------------------------------------------------------------
// Monoids (monoid.py:22-39): identity and pairwise combine.
// ---------------------------------------------------------------------------
template <int M>
struct Mono;
template <>
struct Mono<PLX_MONOID_SUM> {
  static __device__ __forceinline__ float id() { return 0.0f; }
  static __device__ __forceinline__ float op(float a, float b) { return a + b; }
};
template <>
struct Mono<PLX_MONOID_PROD> {
  static __device__ __forceinline__ float id() { return 1.0f; }
  static __device__ __forceinline__ float op(float a, float b) { return a * b; }
};
template <>
struct Mono<PLX_MONOID_MAX> {
  static __device__ __forceinline__ float id() { return -__builtin_huge_valf(); }
  static __device__ __forceinline__ float op(float a, float b) { return px::fmax_nan(a, b); }
};
template <>
struct Mono<PLX_MONOID_MIN> {
  static __device__ __forceinline__ float id() { return __builtin_huge_valf(); }
  static __device__ __forceinline__ float op(float a, float b) { return px::fmin_nan(a, b); }
};

// ---------------------------------------------------------------------------
// Unit-program interpreter. The program is uniform across the grid (it sits
// in the kernel argument segment), so every dispatch below is a scalar branch.
// ---------------------------------------------------------------------------
enum : int32_t {
  OP_ACC = 1, OP_LDU = 2, OP_CONST = 3, OP_ADD = 4, OP_SUB = 5, OP_MUL = 6,
  OP_DIV = 7, OP_NEG = 8, OP_ABS = 9, OP_MAX = 10, OP_MIN = 11, OP_TANH = 12,
  OP_EXP = 13, OP_LOG = 14, OP_SQRT = 15, OP_SIGMOID = 16, OP_GT = 17,
  OP_GE = 18, OP_LT = 19, OP_LE = 20, OP_EQ = 21, OP_NE = 22, OP_SEL = 23,
  OP_OUT = 24, OP_LDX = 25, OP_MOV = 26, OP_SQUARE = 27, OP_RELU = 28,
  OP_SIGN = 29
};

constexpr int kRegs = 16;

// Runs `P` for unit `u`; out slot k is stored to P.outs[k][u] when `store`.
// Returns out slot 1 (the loss term of a loss program).
__device__ float run_program(const plx_program& P, int64_t u, float acc, float aux,
                             bool store) {
  float r[kRegs];
  float outs[PLX_MAX_OUTS];
#pragma unroll
  for (int k = 0; k < kRegs; ++k) r[k] = 0.0f;
#pragma unroll
  for (int k = 0; k < PLX_MAX_OUTS; ++k) outs[k] = 0.0f;
  const int n = P.ninstr;
  for (int k = 0; k < n; ++k) {
    const int op = P.code[4 * k + 0];
    const int dd = P.code[4 * k + 1] & (kRegs - 1);
    const int a = P.code[4 * k + 2];
    const int b = P.code[4 * k + 3];
    const float ra = r[a & (kRegs - 1)];
    const float rb = r[b & (kRegs - 1)];
    float v = 0.0f;
    switch (op) {
      case OP_ACC: v = acc; break;
      case OP_LDU: v = P.fields[a & (PLX_MAX_FIELDS - 1)][u]; break;
      case OP_CONST: v = P.consts[a & (PLX_MAX_CONST - 1)]; break;
      case OP_LDX: v = aux; break;
      case OP_MOV: v = ra; break;
      case OP_ADD: v = ra + rb; break;
      case OP_SUB: v = ra - rb; break;
      case OP_MUL: v = ra * rb; break;
      case OP_DIV: v = ra / rb; break;
      case OP_NEG: v = -ra; break;
      case OP_ABS: v = fabsf(ra); break;
      case OP_SQUARE: v = ra * ra; break;
      case OP_MAX: v = px::fmax_nan(ra, rb); break;
      case OP_MIN: v = px::fmin_nan(ra, rb); break;
      case OP_RELU: v = px::fmax_nan(ra, 0.0f); break;
      case OP_TANH: v = px::tanhf_(ra); break;
      case OP_EXP: v = px::expf_(ra); break;
      case OP_LOG: v = px::logf_(ra); break;
      case OP_SQRT: v = sqrtf(ra); break;
      case OP_SIGMOID: v = px::sigmoidf_(ra); break;
      case OP_SIGN: v = ra > 0.0f ? 1.0f : (ra < 0.0f ? -1.0f : ra); break;
      case OP_GT: v = ra > rb ? 1.0f : 0.0f; break;
      case OP_GE: v = ra >= rb ? 1.0f : 0.0f; break;
      case OP_LT: v = ra < rb ? 1.0f : 0.0f; break;
      case OP_LE: v = ra <= rb ? 1.0f : 0.0f; break;
      case OP_EQ: v = ra == rb ? 1.0f : 0.0f; break;
      case OP_NE: v = ra != rb ? 1.0f : 0.0f; break;
      case OP_SEL: v = ra != 0.0f ? rb : r[(b + 1) & (kRegs - 1)]; break;
      case OP_OUT: outs[P.code[4 * k + 1] & (PLX_MAX_OUTS - 1)] = ra; continue;
      default: continue;
    }
    r[dd] = v;
  }
  if (store) {
    for (int k = 0; k < P.nout; ++k)
      if (P.outs[k]) P.outs[k][u] = outs[k];
  }
  return outs[1];
}

__device__ __forceinline__ bool finalizes(const plx_finalize& f, int u) {
  if (f.fin_level >= 0 && f.level[u] != f.fin_level) return false;
  if (f.skip_inputs && f.is_input[u]) return false;
  if (f.pruned && f.pruned[u]) return false;
  return true;
}

// ---------------------------------------------------------------------------
// Forward: one row (destination unit) per lane. The workgroup's rows own a
// contiguous physical range; it is streamed through LDS in windows of kWin
// terms with 16-byte loads (map = weight * x[src], dead slots contribute the
// identity), and each lane folds its own row from LDS in slot order, carrying
// the running value across windows, so the fold order is the slot order for
// any row length.
// ---------------------------------------------------------------------------
constexpr int kFwdBlock = 256;
#ifndef PLX_FWD_QUADS
#define PLX_FWD_QUADS 8
#endif
constexpr int kWinQuads = PLX_FWD_QUADS;  // 16-byte quads per thread per window
constexpr int kWin = 4 * kWinQuads * kFwdBlock;

template <int M>
__global__ __launch_bounds__(kFwdBlock) void k_forward(plx_forward_desc d) {
  __shared__ float buf[kWin];
  const int row0 = blockIdx.x * kFwdBlock;
  const int r = row0 + threadIdx.x;
  const int rend = min(row0 + kFwdBlock, d.nrows);
  const int e_begin = d.row_ptr[row0];
  const int e_end = d.row_ptr[rend];
  const bool has = r < d.nrows;
  const int my_b = has ? d.row_ptr[r] : 0;
  const int my_e = has ? d.row_ptr[r + 1] : 0;
  const float ident = Mono<M>::id();
  float s = ident;
  for (int w0 = e_begin & ~3; w0 < e_end; w0 += kWin) {
    const int wn = min(kWin, e_end - w0);
    // Issue every load of the window before using any of them.
    int4 sv[kWinQuads];
    float4 wv[kWinQuads];
    uint32_t dv[kWinQuads];
#pragma unroll
    for (int i = 0; i < kWinQuads; ++i) {
      const int q = threadIdx.x + i * kFwdBlock;
      if (4 * q < wn) {
        const int e = w0 + 4 * q;
        sv[i] = *reinterpret_cast<const int4*>(d.src + e);
        wv[i] = *reinterpret_cast<const float4*>(d.weight + e);
        dv[i] = *reinterpret_cast<const uint32_t*>(d.dead + e);
      }
    }
#pragma unroll
    for (int i = 0; i < kWinQuads; ++i) {
      const int q = threadIdx.x + i * kFwdBlock;
      if (4 * q < wn) {
        float4 o;
        o.x = (dv[i] & 0x000000FFu) ? ident : wv[i].x * d.x[sv[i].x];
        o.y = (dv[i] & 0x0000FF00u) ? ident : wv[i].y * d.x[sv[i].y];
        o.z = (dv[i] & 0x00FF0000u) ? ident : wv[i].z * d.x[sv[i].z];
        o.w = (dv[i] & 0xFF000000u) ? ident : wv[i].w * d.x[sv[i].w];
        *reinterpret_cast<float4*>(buf + 4 * q) = o;
      }
    }
    __syncthreads();
    const int lo = max(my_b, w0), hi = min(my_e, w0 + wn);
    for (int e = lo; e < hi; ++e) s = Mono<M>::op(s, buf[e - w0]);
    __syncthreads();
  }
  if (!has) return;
  const int u = d.row_unit[r];
  const float a = Mono<M>::op(d.acc ? d.acc[u] : ident, s);
  if (finalizes(d.fin, u)) {
    run_program(d.apply, u, a, 0.0f, true);
    if (d.acc) d.acc[u] = ident;
  } else if (d.acc) {
    d.acc[u] = a;
  }
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

template <int RULE>
__global__ __launch_bounds__(kUpdBlock) void k_update(plx_update_desc d) {
  const int64_t e = 4 * (static_cast<int64_t>(blockIdx.x) * kUpdBlock + threadIdx.x);
  if (e >= d.n) return;
  const int4 sv = *reinterpret_cast<const int4*>(d.src + e);
  const int4 tv = *reinterpret_cast<const int4*>(d.dst + e);
  const uint32_t dv = *reinterpret_cast<const uint32_t*>(d.dead + e);
  float4 w = *reinterpret_cast<const float4*>(d.weight + e);
  constexpr int nstate = RULE == PLX_RULE_SGD ? 0 : (RULE == PLX_RULE_ADAM ? 3 : 1);
  float4 s0 = make_float4(0.f, 0.f, 0.f, 0.f), s1 = s0, s2 = s0;
  if (nstate >= 1) s0 = *reinterpret_cast<const float4*>(d.s0 + e);
  if (nstate >= 3) {
    s1 = *reinterpret_cast<const float4*>(d.s1 + e);
    s2 = *reinterpret_cast<const float4*>(d.s2 + e);
  }
  if (!(dv & 0x000000FFu)) update_one<RULE>(d, d.gfield[tv.x] * d.act[sv.x], w.x, s0.x, s1.x, s2.x);
  if (!(dv & 0x0000FF00u)) update_one<RULE>(d, d.gfield[tv.y] * d.act[sv.y], w.y, s0.y, s1.y, s2.y);
  if (!(dv & 0x00FF0000u)) update_one<RULE>(d, d.gfield[tv.z] * d.act[sv.z], w.z, s0.z, s1.z, s2.z);
  if (!(dv & 0xFF000000u)) update_one<RULE>(d, d.gfield[tv.w] * d.act[sv.w], w.w, s0.w, s1.w, s2.w);
  *reinterpret_cast<float4*>(d.weight + e) = w;
  if (nstate >= 1) *reinterpret_cast<float4*>(d.s0 + e) = s0;
  if (nstate >= 3) {
    *reinterpret_cast<float4*>(d.s1 + e) = s1;
    *reinterpret_cast<float4*>(d.s2 + e) = s2;
  }
}

// ---------------------------------------------------------------------------
// Backward + update, one destination-sorted tile per workgroup.
//
// The workgroup streams its tile's edge columns once (16-byte loads): for
// each live edge it forms the backward term c = weight * g[dst] with the
// pre-update weight into LDS and, when fused, applies the update rule and
// stores the new weight and optimizer state. Then the tile's (source) groups
// are folded from LDS in physical order -- the group lists are precomputed
// per tile -- and each group sum lands either in the tile's dense row of hot
// partials (sources present in many tiles) or in its slot of the source-major
// cold partial array. No float atomics: every partial has exactly one writer.
// ---------------------------------------------------------------------------
constexpr int kTileBlock = 512;
#ifndef PLX_TILE_QUADS
#define PLX_TILE_QUADS 2
#endif
constexpr int kTileQuads = PLX_TILE_QUADS;  // 16-byte quads per thread per streaming pass

template <int RULE, int M, bool FOLD>
__global__ __launch_bounds__(kTileBlock) void k_tile(plx_tile_desc d) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int T = d.tile_size;
  float* buf = reinterpret_cast<float*>(smem);  // [T]
  float* hot = buf + T;                          // [nhot], padded to 16 bytes
  uint16_t* sl = reinterpret_cast<uint16_t*>(hot + ((d.nhot + 3) & ~3));  // [T]
  const int blk = blockIdx.x;
  const int64_t t0 = d.base + static_cast<int64_t>(blk) * T;
  const int64_t t1 = min(t0 + T, d.end);
  const int n = static_cast<int>(t1 - t0);
  const float ident = Mono<M>::id();
  if (FOLD) {
    for (int j = threadIdx.x; j < d.nhot; j += kTileBlock) hot[j] = ident;
    const uint16_t* slg = d.sorted_local + static_cast<int64_t>(blk) * T;
    for (int j = threadIdx.x; 4 * j < n; j += kTileBlock)
      *reinterpret_cast<uint2*>(sl + 4 * j) = *reinterpret_cast<const uint2*>(slg + 4 * j);
  }
  constexpr int nstate = RULE < 0 || RULE == PLX_RULE_SGD ? 0 : (RULE == PLX_RULE_ADAM ? 3 : 1);
  constexpr int U = kTileQuads;
  // Each pass covers U quads per thread; every load of a pass is issued
  // before any of it is used.
  for (int q0 = threadIdx.x; 4 * q0 < n; q0 += U * kTileBlock) {
    int4 sv[U], tv[U];
    uint32_t dv[U];
    float4 w[U], s0[U], s1[U], s2[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int q = q0 + i * kTileBlock;
      if (4 * q < n) {
        const int64_t e = t0 + 4 * q;
        tv[i] = *reinterpret_cast<const int4*>(d.dst + e);
        dv[i] = *reinterpret_cast<const uint32_t*>(d.dead + e);
        w[i] = *reinterpret_cast<const float4*>(d.weight + e);
        if (RULE >= 0) sv[i] = *reinterpret_cast<const int4*>(d.src + e);
        if (nstate >= 1) s0[i] = *reinterpret_cast<const float4*>(d.s0 + e);
        if (nstate >= 3) {
          s1[i] = *reinterpret_cast<const float4*>(d.s1 + e);
          s2[i] = *reinterpret_cast<const float4*>(d.s2 + e);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int q = q0 + i * kTileBlock;
      if (4 * q >= n) continue;
      const int64_t e = t0 + 4 * q;
      const bool l0 = !(dv[i] & 0x000000FFu), l1 = !(dv[i] & 0x0000FF00u);
      const bool l2 = !(dv[i] & 0x00FF0000u), l3 = !(dv[i] & 0xFF000000u);
      if (FOLD) {
        float4 c;
        c.x = l0 ? w[i].x * d.g[tv[i].x] : ident;
        c.y = l1 ? w[i].y * d.g[tv[i].y] : ident;
        c.z = l2 ? w[i].z * d.g[tv[i].z] : ident;
        c.w = l3 ? w[i].w * d.g[tv[i].w] : ident;
        *reinterpret_cast<float4*>(buf + 4 * q) = c;
      }
      if (RULE >= 0) {
        float4 a = w[i], m = s0[i], v = s1[i], t = s2[i];
        if (l0) update_one<RULE>(d, d.gfield[tv[i].x] * d.act[sv[i].x], a.x, m.x, v.x, t.x);
        if (l1) update_one<RULE>(d, d.gfield[tv[i].y] * d.act[sv[i].y], a.y, m.y, v.y, t.y);
        if (l2) update_one<RULE>(d, d.gfield[tv[i].z] * d.act[sv[i].z], a.z, m.z, v.z, t.z);
        if (l3) update_one<RULE>(d, d.gfield[tv[i].w] * d.act[sv[i].w], a.w, m.w, v.w, t.w);
        *reinterpret_cast<float4*>(d.weight + e) = a;
        if (nstate >= 1) *reinterpret_cast<float4*>(d.s0 + e) = m;
        if (nstate >= 3) {
          *reinterpret_cast<float4*>(d.s1 + e) = v;
          *reinterpret_cast<float4*>(d.s2 + e) = t;
        }
      }
    }
  }
  if (!FOLD) return;
  __syncthreads();
  const int g1 = d.grp_off[blk + 1];
  for (int gi = d.grp_off[blk] + threadIdx.x; gi < g1; gi += kTileBlock) {
    const uint32_t se = d.grp_se[gi];
    const int st = static_cast<int>(se & 0xFFFFu);
    const int len = static_cast<int>(se >> 16);
    float v = ident;
    for (int j = st; j < st + len; ++j) v = Mono<M>::op(v, buf[sl[j]]);
    const int tgt = d.grp_tgt[gi];
    if (tgt >= 0)
      d.cold_partial[tgt] = v;
    else
      hot[-1 - tgt] = v;
  }
  __syncthreads();
  float* hp = d.hot_partial + static_cast<int64_t>(blk) * d.nhot;
  for (int j = threadIdx.x; j < d.nhot; j += kTileBlock) hp[j] = hot[j];
}

// Hot superblock sums: thread (h, superblock) folds the hot partials of the
// superblock's tiles in tile order. Consecutive threads read consecutive
// columns, so every load is coalesced.
template <int M>
__global__ __launch_bounds__(kFwdBlock) void k_hot_sb(plx_partials_desc d) {
  const int h = blockIdx.x * kFwdBlock + threadIdx.x;
  if (h >= d.nhot) return;
  const int sb = blockIdx.y;
  const int k0 = sb * d.superblock;
  const int k1 = min(k0 + d.superblock, d.ntiles);
  const float* hp = d.hot_partial + h;
  float s = Mono<M>::id();
  for (int k = k0; k < k1; ++k) s = Mono<M>::op(s, hp[static_cast<int64_t>(k) * d.nhot]);
  d.hot_sb[static_cast<int64_t>(sb) * d.nhot + h] = s;
}

// Backward finalize from tile partials: one row (source unit) per lane. A hot
// row folds its superblock sums in order; a cold row folds its run of cold
// partials (tile order), closing a superblock sum whenever the superblock id
// changes. Then combine into acc and apply.
template <int M>
__global__ __launch_bounds__(kFwdBlock) void k_partials(plx_partials_desc d) {
  const int r = blockIdx.x * kFwdBlock + threadIdx.x;
  if (r >= d.nrows) return;
  const int u = d.row_unit[r];
  const float ident = Mono<M>::id();
  float s = ident;
  const int h = d.row_hot ? d.row_hot[r] : -1;
  if (h >= 0) {
    const int nsb = (d.ntiles + d.superblock - 1) / d.superblock;
    for (int j = 0; j < nsb; ++j) s = Mono<M>::op(s, d.hot_sb[static_cast<int64_t>(j) * d.nhot + h]);
  } else if (d.row_cold) {
    const int j0 = d.row_cold[r], j1 = d.row_cold[r + 1];
    if (j0 < j1) {
      int cur = d.cold_sb[j0];
      float q = ident;
      for (int j = j0; j < j1; ++j) {
        const int sb = d.cold_sb[j];
        if (sb != cur) {
          s = Mono<M>::op(s, q);
          q = ident;
          cur = sb;
        }
        q = Mono<M>::op(q, d.cold_partial[j]);
      }
      s = Mono<M>::op(s, q);
    }
  }
  const float a = Mono<M>::op(d.acc ? d.acc[u] : ident, s);
  if (finalizes(d.fin, u)) {
    run_program(d.apply, u, a, 0.0f, true);
    if (d.acc) d.acc[u] = ident;
  } else if (d.acc) {
    d.acc[u] = a;
  }
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
__global__ __launch_bounds__(kPiece) void k_loss_pieces(int32_t n_out, const int32_t* ids,
                                                       const float* targets, plx_program P,
                                                       float* piece_sums) {
  __shared__ float terms[kPiece];
  const int k = blockIdx.x * kPiece + threadIdx.x;
  if (k < n_out) terms[threadIdx.x] = run_program(P, ids[k], 0.0f, targets[k], true);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int len = min(kPiece, n_out - static_cast<int>(blockIdx.x) * kPiece);
    float s = 0.0f;
    for (int j = 0; j < len; ++j) s = s + terms[j];
    piece_sums[blockIdx.x] = s;
  }
}

// Folds n piece sums in order from +0.0 into *out, staging them through LDS.
__global__ __launch_bounds__(1024) void k_fold_sums(int32_t n, const float* sums, float* out) {
  __shared__ float buf[1024];
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

__global__ __launch_bounds__(1024) void k_softmax_ce(int32_t n, const int32_t* ids,
                                                     const float* act, const float* targets,
                                                     float* seed_field, float* loss_out) {
  __shared__ float red[1024];
  __shared__ float piece[kSoftmaxMaxPieces];
  __shared__ float bcast[2];
  const int tid = threadIdx.x;
  // 1. max by a '>' scan from -inf (NaN is never taken), then a tree.
  float m = -__builtin_huge_valf();
  for (int k = tid; k < n; k += blockDim.x) {
    const float a = act[ids[k]];
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
    for (int k = p * kPiece; k < end; ++k) s = s + px::expf_(act[ids[k]] - peak);
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
      const float z = act[ids[k]] - peak;
      const float t = targets[k];
      seed_field[ids[k]] = px::expf_(z) / total - t;
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

__device__ __forceinline__ uint32_t philox32_dev(uint64_t seed, uint64_t counter) {
  uint32_t x0 = static_cast<uint32_t>(counter), x1 = static_cast<uint32_t>(counter >> 32);
  uint32_t x2 = static_cast<uint32_t>(seed), x3 = static_cast<uint32_t>(seed >> 32);
  uint32_t k0 = x2, k1 = x3;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = 0xD2511F53u * x0, hi0 = __umulhi(0xD2511F53u, x0);
    const uint32_t lo1 = 0xCD9E8D57u * x2, hi1 = __umulhi(0xCD9E8D57u, x2);
    const uint32_t n0 = hi1 ^ x1 ^ k0, n2 = hi0 ^ x3 ^ k1;
    x0 = n0;
    x1 = lo1;
    x2 = n2;
    x3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return x0;
}

__global__ void k_philox(int64_t n, const uint64_t* seeds, const uint64_t* ctrs, uint32_t* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = philox32_dev(seeds[i], ctrs[i]);
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
    default: r = px::pow_step(v, y[i]); break;
  }
  out[i] = r;
}

inline unsigned grid_for(int64_t n, int block) {
  return static_cast<unsigned>((n + block - 1) / block);
}

bool program_ok(const plx_program& p) {
  return p.ninstr >= 0 && p.ninstr <= PLX_MAX_INSTR && p.nout >= 0 && p.nout <= PLX_MAX_OUTS;
}

template <int RULE, int M, bool FOLD>
void launch_tile(const plx_tile_desc& d, size_t lds, hipStream_t s) {
  // LDS beyond 64 KiB needs an explicit per-kernel opt-in.
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&k_tile<RULE, M, FOLD>),
      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  (void)attr;
  k_tile<RULE, M, FOLD><<<d.ntiles, kTileBlock, lds, s>>>(d);
}

template <int M, bool FOLD>
int dispatch_rule(const plx_tile_desc& d, size_t lds, hipStream_t s) {
  switch (d.update ? d.rule : -1) {
    case -1: launch_tile<-1, M, FOLD>(d, lds, s); break;
    case PLX_RULE_SGD: launch_tile<PLX_RULE_SGD, M, FOLD>(d, lds, s); break;
    case PLX_RULE_MOMENTUM: launch_tile<PLX_RULE_MOMENTUM, M, FOLD>(d, lds, s); break;
    case PLX_RULE_ADAM: launch_tile<PLX_RULE_ADAM, M, FOLD>(d, lds, s); break;
    case PLX_RULE_RMSPROP: launch_tile<PLX_RULE_RMSPROP, M, FOLD>(d, lds, s); break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_backward_tiles: unknown rule");
  }
  return PLX_OK;
}

}  // namespace

extern "C" {

const char* plx_last_error(void) { return g_last_error.c_str(); }

int32_t plx_abi_version(void) { return 1; }

int plx_struct_sizes(int64_t* out, int32_t n) {
  const int64_t sizes[6] = {
      sizeof(plx_program),          sizeof(plx_finalize),
      sizeof(plx_forward_desc),     sizeof(plx_tile_desc),
      sizeof(plx_partials_desc),    sizeof(plx_update_desc)};
  for (int32_t k = 0; k < n && k < 6; ++k) out[k] = sizes[k];
  return 6;
}

int plx_forward_bucket(const plx_forward_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_forward_bucket: null descriptor");
  if (d->nrows < 0) return fail(PLX_ERR_INVALID, "plx_forward_bucket: negative nrows");
  if (d->nrows == 0) return PLX_OK;
  if (!d->row_unit || !d->row_ptr || !d->src || !d->weight || !d->dead || !d->x)
    return fail(PLX_ERR_INVALID, "plx_forward_bucket: null column");
  if (!program_ok(d->apply)) return fail(PLX_ERR_INVALID, "plx_forward_bucket: bad program");
  if (d->fin.fin_level >= 0 && !d->fin.level)
    return fail(PLX_ERR_INVALID, "plx_forward_bucket: level needed");
  if (d->fin.skip_inputs && !d->fin.is_input)
    return fail(PLX_ERR_INVALID, "plx_forward_bucket: is_input needed");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(d->nrows, kFwdBlock);
  switch (d->monoid) {
    case PLX_MONOID_SUM: k_forward<PLX_MONOID_SUM><<<grid, kFwdBlock, 0, s>>>(*d); break;
    case PLX_MONOID_PROD: k_forward<PLX_MONOID_PROD><<<grid, kFwdBlock, 0, s>>>(*d); break;
    case PLX_MONOID_MAX: k_forward<PLX_MONOID_MAX><<<grid, kFwdBlock, 0, s>>>(*d); break;
    case PLX_MONOID_MIN: k_forward<PLX_MONOID_MIN><<<grid, kFwdBlock, 0, s>>>(*d); break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_forward_bucket: unknown monoid");
  }
  return check_launch("plx_forward_bucket");
}

int plx_backward_tiles(const plx_tile_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_backward_tiles: null descriptor");
  if (d->ntiles < 0 || d->tile_size <= 0 || d->tile_size % 4 || d->tile_size > 32768)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: tile_size must be a positive multiple of 4 <= 32768");
  if (d->base % 4 || d->end % 4 || d->end < d->base)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: base/end must be multiples of 4");
  if ((d->end - d->base + d->tile_size - 1) / d->tile_size != d->ntiles)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: ntiles does not cover [base, end)");
  if (d->ntiles == 0) return PLX_OK;
  if (!d->src || !d->dst || !d->dead || !d->weight)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: null column");
  if (d->fold && (!d->grp_off || !d->grp_se || !d->grp_tgt || !d->sorted_local || !d->g ||
                  (d->nhot > 0 && !d->hot_partial)))
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: fold metadata missing");
  if (d->update && (!d->gfield || !d->act))
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: update fields missing");
  if (d->update && (d->rule == PLX_RULE_MOMENTUM || d->rule == PLX_RULE_RMSPROP) && !d->s0)
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: state column missing");
  if (d->update && d->rule == PLX_RULE_ADAM && (!d->s0 || !d->s1 || !d->s2))
    return fail(PLX_ERR_INVALID, "plx_backward_tiles: Adam state columns missing");
  if (!d->fold && !d->update) return PLX_OK;
  if (d->fold && d->nhot < 0) return fail(PLX_ERR_INVALID, "plx_backward_tiles: negative nhot");
  const size_t lds = d->fold ? static_cast<size_t>(d->tile_size) * 6 +
                                   static_cast<size_t>((d->nhot + 3) & ~3) * 4
                             : 0;
  if (lds > 160 * 1024) return fail(PLX_ERR_UNSUPPORTED, "plx_backward_tiles: tile does not fit in LDS");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = PLX_OK;
  if (!d->fold) {
    rc = dispatch_rule<PLX_MONOID_SUM, false>(*d, 0, s);
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
  if (d->row_hot && (d->nhot < 0 || d->superblock <= 0 || d->ntiles < 0 ||
                     (d->nhot > 0 && (!d->hot_partial || !d->hot_sb))))
    return fail(PLX_ERR_INVALID, "plx_backward_partials: hot partials missing");
  if (d->row_cold && (!d->cold_partial || !d->cold_sb))
    return fail(PLX_ERR_INVALID, "plx_backward_partials: cold partials missing");
  if (!program_ok(d->apply)) return fail(PLX_ERR_INVALID, "plx_backward_partials: bad program");
  if (d->fin.fin_level >= 0 && !d->fin.level)
    return fail(PLX_ERR_INVALID, "plx_backward_partials: level needed");
  if (d->fin.skip_inputs && !d->fin.is_input)
    return fail(PLX_ERR_INVALID, "plx_backward_partials: is_input needed");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (d->row_hot && d->nhot > 0 && d->ntiles > 0) {
    const dim3 g(grid_for(d->nhot, kFwdBlock), (d->ntiles + d->superblock - 1) / d->superblock);
    switch (d->monoid) {
      case PLX_MONOID_SUM: k_hot_sb<PLX_MONOID_SUM><<<g, kFwdBlock, 0, s>>>(*d); break;
      case PLX_MONOID_PROD: k_hot_sb<PLX_MONOID_PROD><<<g, kFwdBlock, 0, s>>>(*d); break;
      case PLX_MONOID_MAX: k_hot_sb<PLX_MONOID_MAX><<<g, kFwdBlock, 0, s>>>(*d); break;
      case PLX_MONOID_MIN: k_hot_sb<PLX_MONOID_MIN><<<g, kFwdBlock, 0, s>>>(*d); break;
      default: return fail(PLX_ERR_UNSUPPORTED, "plx_backward_partials: unknown monoid");
    }
    const int rc = check_launch("plx_backward_partials");
    if (rc) return rc;
  }
  const unsigned grid = grid_for(d->nrows, kFwdBlock);
  switch (d->monoid) {
    case PLX_MONOID_SUM: k_partials<PLX_MONOID_SUM><<<grid, kFwdBlock, 0, s>>>(*d); break;
    case PLX_MONOID_PROD: k_partials<PLX_MONOID_PROD><<<grid, kFwdBlock, 0, s>>>(*d); break;
    case PLX_MONOID_MAX: k_partials<PLX_MONOID_MAX><<<grid, kFwdBlock, 0, s>>>(*d); break;
    case PLX_MONOID_MIN: k_partials<PLX_MONOID_MIN><<<grid, kFwdBlock, 0, s>>>(*d); break;
    default: return fail(PLX_ERR_UNSUPPORTED, "plx_backward_partials: unknown monoid");
  }
  return check_launch("plx_backward_partials");
}

int plx_update_conn(const plx_update_desc* d, void* stream) {
  if (!d) return fail(PLX_ERR_INVALID, "plx_update_conn: null descriptor");
  if (d->n < 0) return fail(PLX_ERR_INVALID, "plx_update_conn: negative n");
  if (d->n == 0) return PLX_OK;
  if (d->n % 4 != 0) return fail(PLX_ERR_INVALID, "plx_update_conn: n must be a multiple of 4");
  if (!d->src || !d->dst || !d->dead || !d->weight || !d->gfield || !d->act)
    return fail(PLX_ERR_INVALID, "plx_update_conn: null column");
  if ((d->rule == PLX_RULE_MOMENTUM || d->rule == PLX_RULE_RMSPROP) && !d->s0)
    return fail(PLX_ERR_INVALID, "plx_update_conn: state column missing");
  if (d->rule == PLX_RULE_ADAM && (!d->s0 || !d->s1 || !d->s2))
    return fail(PLX_ERR_INVALID, "plx_update_conn: Adam state columns missing");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(d->n / 4, kUpdBlock);
  switch (d->rule) {
    case PLX_RULE_SGD: k_update<PLX_RULE_SGD><<<grid, kUpdBlock, 0, s>>>(*d); break;
    case PLX_RULE_MOMENTUM: k_update<PLX_RULE_MOMENTUM><<<grid, kUpdBlock, 0, s>>>(*d); break;
    case PLX_RULE_ADAM: k_update<PLX_RULE_ADAM><<<grid, kUpdBlock, 0, s>>>(*d); break;
    case PLX_RULE_RMSPROP: k_update<PLX_RULE_RMSPROP><<<grid, kUpdBlock, 0, s>>>(*d); break;
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
  if (!program_ok(*term)) return fail(PLX_ERR_INVALID, "plx_loss_elementwise: bad program");
  if (n_out > 0 && (!output_ids || !targets || !seed_field))
    return fail(PLX_ERR_INVALID, "plx_loss_elementwise: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  plx_program p = *term;
  p.outs[0] = seed_field;  // slot 0: the seed, stored at the output unit
  p.outs[1] = nullptr;     // slot 1: the term, returned to the kernel
  if (p.nout < 2) p.nout = 2;
  const int npieces = (n_out + kPiece - 1) / kPiece;
  if (npieces > 0) {
    k_loss_pieces<<<npieces, kPiece, 0, s>>>(n_out, output_ids, targets, p, partials);
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
                                                                  targets, seed_field, loss_out);
  return check_launch("plx_loss_softmax_ce");
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
  if (n < 0 || op < 0 || op > 5) return fail(PLX_ERR_INVALID, "plx_eval_math: bad argument");
  if (n == 0) return PLX_OK;
  if (!x || !out || (op == 5 && !y)) return fail(PLX_ERR_INVALID, "plx_eval_math: null pointer");
  k_math<<<grid_for(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(op, n, x, y, out);
  return check_launch("plx_eval_math");
}

}  // extern "C"
