// px_forward.h -- the forward sweep of one bucket (k_forward's body) and the
// device pieces it shares with the library's other edge kernels: streaming
// loads, monoids, the unit-program interpreter, LDS source tables.
//
// Compiled twice: into the library (plastax_hip.hip: k_forward, the PruneConn
// predicate, when there is one, interpreted per position) and by hipRTC for a
// fused forward + PruneConn whose predicate is compiled in
// (plx_forward_prune_compile: the program's instructions as straight-line
// code, the same operations in the same order, so both give the same bits).
#pragma once

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

#include "../../include/plastax_hip.h"
#include "px_common.h"
#include "px_math.h"
#include "px_site.h"

namespace {

// Streaming (non-temporal) 16-byte accesses for the edge columns: each
// position is read and written once per pass, so these lines should not
// displace the gathered unit vectors and partials in the caches.
typedef float nt_v4f __attribute__((ext_vector_type(4)));
typedef int nt_v4i __attribute__((ext_vector_type(4)));
typedef unsigned nt_v2u __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 ld_stream(const float* p) {
  const nt_v4f v = __builtin_nontemporal_load(reinterpret_cast<const nt_v4f*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ int4 ld_stream(const int32_t* p) {
  const nt_v4i v = __builtin_nontemporal_load(reinterpret_cast<const nt_v4i*>(p));
  return make_int4(v.x, v.y, v.z, v.w);
}
// One-byte destinations (dst8): TO_ID = blk_dst0[rel >> kDst8Shift] + dst8[rel]
// for a bucket-relative position rel.
constexpr int kDst8Shift = 12;

__device__ __forceinline__ uint32_t ld_stream(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}
__device__ __forceinline__ uint2 ld_stream(const uint16_t* p) {
  const nt_v2u v = __builtin_nontemporal_load(reinterpret_cast<const nt_v2u*>(p));
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ void st_stream(float* p, float4 a) {
  const nt_v4f v = {a.x, a.y, a.z, a.w};
  __builtin_nontemporal_store(v, reinterpret_cast<nt_v4f*>(p));
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

// A map's term: (connection factor) * (unit factor), each the loaded value
// or the map's constant (plx_map; the flags are uniform, so these are
// scalar selects).
__device__ __forceinline__ float map_term(const plx_map& m, float w, float x) {
  return ((m.flags & PLX_MAP_W_CONST) ? m.w : w) * ((m.flags & PLX_MAP_X_CONST) ? m.x : x);
}

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
  OP_SIGN = 29, OP_LOG1P = 30, OP_EXPM1 = 31, OP_COS = 33, OP_SIN = 34
};

constexpr int kRegs = 16;

// The unit fields a program reads (LDU), loaded for one unit ahead of time:
// a program reads its fields only at its own unit, so every load can be
// issued before the work that produces `acc`.
struct UnitFields {
  float v[PLX_MAX_FIELDS];
};

// Field k of `f`; k is uniform across the wave, so this is a scalar branch
// and the values stay in registers.
__device__ __forceinline__ float pick_field(const UnitFields& f, int k) {
  switch (k & (PLX_MAX_FIELDS - 1)) {
    case 0: return f.v[0];
    case 1: return f.v[1];
    case 2: return f.v[2];
    case 3: return f.v[3];
    case 4: return f.v[4];
    case 5: return f.v[5];
    case 6: return f.v[6];
    default: return f.v[7];
  }
}

// Loads the program's fields at unit u: a uniform switch on the field count
// leaves straight-line code with every load issued before any is used.
__device__ __forceinline__ UnitFields load_fields(const plx_program& P, int64_t u) {
  UnitFields f;
#pragma unroll
  for (int k = 0; k < PLX_MAX_FIELDS; ++k) f.v[k] = 0.0f;
  switch (P.nfields) {
    case 8: f.v[7] = P.fields[7][u]; [[fallthrough]];
    case 7: f.v[6] = P.fields[6][u]; [[fallthrough]];
    case 6: f.v[5] = P.fields[5][u]; [[fallthrough]];
    case 5: f.v[4] = P.fields[4][u]; [[fallthrough]];
    case 4: f.v[3] = P.fields[3][u]; [[fallthrough]];
    case 3: f.v[2] = P.fields[2][u]; [[fallthrough]];
    case 2: f.v[1] = P.fields[1][u]; [[fallthrough]];
    case 1: f.v[0] = P.fields[0][u]; [[fallthrough]];
    default: break;
  }
  return f;
}

// A loss program's fields at output row u of sample b: a field whose
// fixed_mask bit is set points at one fixed unit's row and is read at b.
__device__ __forceinline__ UnitFields load_loss_fields(const plx_program& P, int64_t u, int b) {
  UnitFields f;
#pragma unroll
  for (int k = 0; k < PLX_MAX_FIELDS; ++k)
    f.v[k] = k < P.nfields ? P.fields[k][(P.fixed_mask >> k) & 1 ? static_cast<int64_t>(b) : u] : 0.0f;
  return f;
}

// Runs `P` for unit `u`, reading its fields from `f`; out slot k is stored to
// P.outs[k][u] when `store`. Returns out slot 1 (the loss term of a loss
// program).
__device__ __forceinline__ float run_program(const plx_program& P, int64_t u, const UnitFields& f, float acc,
                             float aux, bool store) {
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
      case OP_LDU: v = pick_field(f, a); break;
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
      case OP_COS: v = px::cosf_(ra); break;
      case OP_SIN: v = px::sinf_(ra); break;
      case OP_LOG1P: v = px::log1pf_(ra); break;
      case OP_EXPM1: v = px::expm1f_(ra); break;
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

// Whether unit u finalizes. level and is_input are never null (the entry
// points check); a null `pruned` reads is_input and is masked off, so the
// three loads are unconditional and issued before any is tested.
__device__ __forceinline__ bool finalizes(const plx_finalize& f, int u) {
  const int lv = f.level[u];
  const int inp = f.is_input[u];
  const int prn = (f.pruned ? f.pruned : f.is_input)[u];
  return (f.fin_level < 0 || lv == f.fin_level) && !(f.skip_inputs && inp) &&
         !(f.pruned && prn);
}

// A row's unit, whether it finalizes and the fields its program reads,
// loaded together before the row's reduction.
struct RowPre {
  int u;
  bool fin;
  UnitFields f;
};

__device__ __forceinline__ RowPre prefetch_row(const int32_t* row_unit, int r,
                                               const plx_finalize& fin,
                                               const plx_program& P) {
  RowPre p;
  p.u = row_unit[r];
  p.fin = finalizes(fin, p.u);
  p.f = load_fields(P, p.u);
  return p;
}

// ---------------------------------------------------------------------------
// Source-value tables. Units are numbered most-used source first within each
// level, so the values a bucket gathers most are one contiguous slice
// x[base, base + len); a workgroup copies it into LDS once and gathers those
// sources from there (the same bits, without an L1/L2 request per lane).
// ---------------------------------------------------------------------------
constexpr int kTbl = PLX_MAX_TBL;

// Copies x[base, base + len) into tbl with every load issued before any LDS
// store (len <= CAP; the caller synchronises before use).
template <int BLOCK, int CAP = kTbl>
__device__ __forceinline__ void stage_table(float* tbl, const float* x, int base, int len) {
  if (len <= 0) return;
  constexpr int kPer = CAP > 0 ? (CAP + BLOCK - 1) / BLOCK : 1;
  float v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) v[i] = x[base + min(static_cast<int>(threadIdx.x) + i * BLOCK, len - 1)];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = threadIdx.x + i * BLOCK;
    if (j < len) tbl[j] = v[i];
  }
}

// Gathers K values x[idx[k]] (lanes with use[k] false read the table's first
// entry, or x[0] without a table, and their value is ignored): table hits
// read LDS, the rest issue one global load each, all before any is used.
// A hit and a miss share out[k], so the table read waits for the global
// loads in flight (the memory counter retires in order); gather_split
// keeps them apart.
template <int K>
__device__ __forceinline__ void gather_k(const float* tbl, const float* x, int base, int len,
                                         const int* idx, const bool* use, float* out) {
  int o[K];
  bool in[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int i = use[k] ? idx[k] : (len > 0 ? base : 0);
    o[k] = i - base;
    in[k] = static_cast<unsigned>(o[k]) < static_cast<unsigned>(len);
    if (!in[k]) out[k] = x[i];
  }
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (in[k]) out[k] = tbl[o[k]];
}

// As gather_k, with table hits read into hit[k] and misses into miss[k]
// (the register of the other kind holds 0): the value is
// gather_join(hit[k], miss[k]), taken where it is used, so nothing here
// waits for the global loads.
template <int K>
__device__ __forceinline__ void gather_split(const float* tbl, const float* x, int base, int len,
                                             const int* idx, const bool* use, uint32_t* hit, uint32_t* miss) {
  int o[K];
  bool in[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int i = use[k] ? idx[k] : (len > 0 ? base : 0);
    o[k] = i - base;
    in[k] = static_cast<unsigned>(o[k]) < static_cast<unsigned>(len);
    miss[k] = 0u;
    if (!in[k]) miss[k] = __float_as_uint(x[i]);
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    hit[k] = 0u;
    if (in[k]) hit[k] = __float_as_uint(tbl[o[k]]);
  }
}

__device__ __forceinline__ float gather_join(uint32_t hit, uint32_t miss) { return __uint_as_float(hit | miss); }

// A launch-uniform read of a layout table through the scalar cache (the
// constant address space: the tables are written by earlier launches and
// only read by the kernels that use this). Waiting for a scalar load does
// not wait for the vector loads and stores in flight, which retire in order.
typedef const __attribute__((address_space(4))) int32_t const_i32;
__device__ __forceinline__ int32_t ld_uniform(const int32_t* p, int64_t i) {
  return ((const_i32*)p)[i];
}

// ---------------------------------------------------------------------------
// Forward: rows (destination units) are cut into blocks of kFwdRows, one row
// per lane of the first kFwdRows lanes. Each workgroup of a persistent grid
// (kFwdPerCU per CU) takes a contiguous run of blocks, whose positions are
// contiguous too, and streams them through LDS in windows of kFwdWin terms
// with 16-byte loads of FROM_ID and WEIGHT (map = weight * x[src], table hits
// read LDS). Each row's lane folds its terms from LDS in slot order, carrying
// the running value across windows, so the fold order is the slot order for
// any row length. The next window's loads (at a block's end, the next
// block's first window) are issued before the current window is folded, so
// the fold and the row finalize never leave the memory system idle. Row
// ranges cover live positions only; DEAD is read only when the caller passes
// it (a bucket with tombstones inside its rows).
// ---------------------------------------------------------------------------
#ifndef PLX_FWD_BLOCK
#define PLX_FWD_BLOCK 512
#endif
#ifndef PLX_FWD_ROWS
#define PLX_FWD_ROWS 256
#endif
#ifndef PLX_FWD_TBL
#define PLX_FWD_TBL 8192
#endif
#ifndef PLX_FWD_QUADS
#define PLX_FWD_QUADS 2
#endif
#ifndef PLX_FWD_PER_CU
#define PLX_FWD_PER_CU 2
#endif
constexpr int kFwdBlock = PLX_FWD_BLOCK;
constexpr int kFwdRows = PLX_FWD_ROWS;  // rows per block, one lane each
static_assert(kFwdRows <= kFwdBlock, "a block's rows need a lane each");
constexpr int kFwdTbl = PLX_FWD_TBL;
constexpr int kFwdQuads = PLX_FWD_QUADS;  // 16-byte quads per thread per window
constexpr int kFwdWin = 4 * kFwdQuads * kFwdBlock;
constexpr int kFwdPerCU = PLX_FWD_PER_CU;  // workgroups per CU in the persistent grid

// A window's raw columns: FROM_ID and WEIGHT quads, DEAD bytes.
struct FwdRaw {
  int4 sv[kFwdQuads];
  float4 wv[kFwdQuads];
  uint32_t dv[kFwdQuads];
};

// A window: positions [w0, w0 + kFwdWin) of block b, whose rows own [eb, ee).
struct FwdWin {
  int b, w0, eb, ee;
};

// The fused forward's PruneConn predicate at position p (an EDGE site of
// the bucket's positions, as plx_site_eval runs it on the physical arena);
// Prog runs the program (SiteInterp, or a compiled program's SiteGen).
template <class Prog>
__device__ __forceinline__ uint8_t prune_at(const plx_forward_desc& d, int64_t p, uint32_t keyed) {
  Site c;
  c.role[0] = c.role[1] = c.role[2] = c.role[3] = 0;
  const int32_t s = static_cast<int32_t>(p - d.prune_base);
  c.role[4] = s;
  c.cid_value = d.prune_slot ? d.prune_slot[s] : s;
  c.seed = static_cast<uint64_t>(keyed) << 32;
  c.ids_logical = d.ids_logical;
  c.ids_physical = d.ids_physical;
  c.batch = 1;
  c.sample = 0;
  uint32_t out[PLX_MAX_SOUTS];
  out[0] = 0;
  Prog::run(*d.prune_prog, c, d.num_units, out);
  return out[0] != 0u;
}

// The body of a forward launch (kFwdBlock lanes per workgroup). PRUNE: the
// PruneConn predicate of every visited position goes to prune_sink (see
// plx_forward_desc), evaluated by Prog.
template <int M, bool PRUNE, class Prog>
__device__ __forceinline__ void forward_body(const plx_forward_desc& d) {
  __shared__ __align__(16) float buf[2][kFwdWin];
  __shared__ float tbl[kFwdTbl > 0 ? kFwdTbl : 1];
  const int nblk = (d.nrows + kFwdRows - 1) / kFwdRows;
  const int b0 = static_cast<int>(static_cast<int64_t>(blockIdx.x) * nblk / gridDim.x);
  const int b1 = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * nblk / gridDim.x);
  if (b0 >= b1) return;  // uniform over the workgroup
  const int tlen = kFwdTbl > 0 ? min(d.tbl_len, kFwdTbl) : 0;
  const float ident = Mono<M>::id();
  auto row_end = [&](int blk) { return d.row_ptr[min((blk + 1) * kFwdRows, d.nrows)]; };

  // Windows in order: every block has at least one (an empty block's
  // window holds nothing). ee_next is the end of the block after the last
  // window handed out.
  int ee_next = b0 + 1 < b1 ? row_end(b0 + 1) : 0;
  auto next_win = [&](const FwdWin& w) {
    FwdWin n = w;
    n.w0 = w.w0 + kFwdWin;
    if (n.w0 >= w.ee) {
      n.b = w.b + 1;
      n.eb = w.ee;
      n.ee = ee_next;
      n.w0 = n.eb & ~3;
      if (n.b + 1 < b1) ee_next = row_end(n.b + 1);
    }
    return n;
  };
  auto load = [&](FwdRaw& R, const FwdWin& w) {
#pragma unroll
    for (int i = 0; i < kFwdQuads; ++i) {
      const int q = threadIdx.x + i * kFwdBlock;
      R.dv[i] = 0;
      if (w.w0 + 4 * q < w.ee) {
        const int e = w.w0 + 4 * q;
        R.sv[i] = ld_stream(d.src + e);
        R.wv[i] = ld_stream(d.weight + e);
        if (d.dead) R.dv[i] = *reinterpret_cast<const uint32_t*>(d.dead + e);
      }
    }
  };
  // Terms of window w from its raw columns into out; the loads of window
  // `ahead` into `spare` go out between the gathers and their use. Only
  // positions of the window's block rows contribute.
  auto terms = [&](const FwdRaw& cur, const FwdWin& w, float* out, FwdRaw& spare, const FwdWin& ahead,
                   bool load_ahead) {
    const int wn = min(kFwdWin, w.ee - w.w0);
    bool ok[kFwdQuads][4];
    float xv[kFwdQuads][4];
#pragma unroll
    for (int i = 0; i < kFwdQuads; ++i) {
      const int e = w.w0 + 4 * (threadIdx.x + i * kFwdBlock);
      const bool in = 4 * (threadIdx.x + i * kFwdBlock) < wn;
      const int idx[4] = {cur.sv[i].x, cur.sv[i].y, cur.sv[i].z, cur.sv[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k)
        ok[i][k] = in && e + k >= w.eb && e + k < w.ee && !((cur.dv[i] >> (8 * k)) & 0xFFu);
      gather_k<4>(tbl, d.x, d.tbl_base, tlen, idx, ok[i], xv[i]);
    }
    if (load_ahead) load(spare, ahead);
#pragma unroll
    for (int i = 0; i < kFwdQuads; ++i) {
      const int q = threadIdx.x + i * kFwdBlock;
      if (4 * q < wn) {
        float4 o;
        o.x = ok[i][0] ? map_term(d.map, cur.wv[i].x, xv[i][0]) : ident;
        o.y = ok[i][1] ? map_term(d.map, cur.wv[i].y, xv[i][1]) : ident;
        o.z = ok[i][2] ? map_term(d.map, cur.wv[i].z, xv[i][2]) : ident;
        o.w = ok[i][3] ? map_term(d.map, cur.wv[i].w, xv[i][3]) : ident;
        *reinterpret_cast<float4*>(out + 4 * q) = o;
      }
    }
    if (PRUNE) {
      // Each position of the rows' ranges is in exactly one window's
      // [eb, ee), so every sink byte has one writer.
      const uint32_t keyed = px::philox32(0, 1);  // the rng key of an unseeded step-0 site
      if constexpr (Prog::kSites > 1) {
        // A compiled program: the thread's positions evaluated together (a
        // position outside the rows' ranges evaluates the nearest one and
        // stores nothing), so all their loads are in flight at once.
        if (w.ee <= w.eb) return;
        uint8_t kill[kFwdQuads][4];
#pragma unroll
        for (int i = 0; i < kFwdQuads; ++i) {
          const int q = threadIdx.x + i * kFwdBlock;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int p = w.w0 + 4 * q + k;
            kill[i][k] = prune_at<Prog>(d, p < w.eb ? w.eb : (p >= w.ee ? w.ee - 1 : p), keyed);
          }
        }
#pragma unroll
        for (int i = 0; i < kFwdQuads; ++i) {
          const int q = threadIdx.x + i * kFwdBlock;
          if (4 * q >= wn) continue;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int p = w.w0 + 4 * q + k;
            if (p < w.eb || p >= w.ee) continue;
            d.prune_sink[p] = ((cur.dv[i] >> (8 * k)) & 0xFFu) ? 0 : kill[i][k];
          }
        }
        return;
      }
      // The interpreter: one rolled loop over the thread's positions, a
      // single inlined copy of it (unrolled, each copy adds its registers).
#pragma unroll 1
      for (int t = 0; t < 4 * kFwdQuads; ++t) {
        const int i = t >> 2, k = t & 3;
        const int q = threadIdx.x + i * kFwdBlock;
        const int p = w.w0 + 4 * q + k;
        if (4 * q >= wn || p < w.eb || p >= w.ee) continue;
        uint32_t dv = static_cast<uint32_t>(cur.dv[0]);
#pragma unroll
        for (int ii = 1; ii < kFwdQuads; ++ii)
          if (i == ii) dv = static_cast<uint32_t>(cur.dv[ii]);
        const bool tomb = (dv >> (8 * k)) & 0xFFu;
        d.prune_sink[p] = tomb ? 0 : prune_at<Prog>(d, p, keyed);
      }
    }
  };

  // The rows being folded (block fb): lane's row r, its positions [my_b, my_e).
  int fb = b0;
  int r = 0, my_b = 0, my_e = 0;
  bool has = false;
  RowPre pre;
  auto setup_rows = [&]() {
    r = fb * kFwdRows + static_cast<int>(threadIdx.x);
    has = threadIdx.x < kFwdRows && r < d.nrows;
    my_b = has ? d.row_ptr[r] : 0;
    my_e = has ? d.row_ptr[r + 1] : 0;
    if (has) pre = prefetch_row(d.row_unit, r, d.fin, d.apply);
  };
  float s = ident;
  // The lane's row over window w held in `in`: the unaligned head one term
  // at a time, then aligned 16-byte runs, the last one padded with the
  // identity past the row's end (for every monoid that leaves the running
  // value's bits unchanged: a sum that starts at +0 never holds -0).
  auto fold = [&](const float* in, const FwdWin& w) {
    const int wn = min(kFwdWin, w.ee - w.w0);
    const int lo = max(my_b, w.w0) - w.w0;
    const int hi = min(my_e, w.w0 + wn) - w.w0;
    if (lo >= hi) return;
    int j = lo;
    const int a = min((lo + 3) & ~3, hi);
    for (; j < a; ++j) s = Mono<M>::op(s, in[j]);
    for (; j + 8 <= hi; j += 8) {
      const float4 x0 = *reinterpret_cast<const float4*>(in + j);
      const float4 x1 = *reinterpret_cast<const float4*>(in + j + 4);
      s = Mono<M>::op(s, x0.x);
      s = Mono<M>::op(s, x0.y);
      s = Mono<M>::op(s, x0.z);
      s = Mono<M>::op(s, x0.w);
      s = Mono<M>::op(s, x1.x);
      s = Mono<M>::op(s, x1.y);
      s = Mono<M>::op(s, x1.z);
      s = Mono<M>::op(s, x1.w);
    }
    for (; j < hi; j += 4) {
      const float4 x = *reinterpret_cast<const float4*>(in + j);
      s = Mono<M>::op(s, x.x);
      s = Mono<M>::op(s, j + 1 < hi ? x.y : ident);
      s = Mono<M>::op(s, j + 2 < hi ? x.z : ident);
      s = Mono<M>::op(s, j + 3 < hi ? x.w : ident);
    }
  };

  // Prologue: window 0's loads, the table, the first rows, window 0's
  // terms (window 1's loads go out meanwhile).
  FwdWin wc{b0, 0, d.row_ptr[b0 * kFwdRows], row_end(b0)};
  wc.w0 = wc.eb & ~3;
  FwdRaw A, B;
  load(A, wc);
  stage_table<kFwdBlock, (kFwdTbl > 0 ? kFwdTbl : 1)>(tbl, d.x, d.tbl_base, tlen);
  setup_rows();
  __syncthreads();
  FwdWin wn1 = next_win(wc);
  terms(A, wc, buf[0], B, wn1, wn1.b < b1);
  __syncthreads();
  // Step k: window k+1's terms (window k+2's loads go out meanwhile) and
  // window k's fold in the same phase, one barrier each. `cur` holds window
  // k+1's loads and `spare` receives window k+2's.
  int par = 0;
  auto step = [&](FwdRaw& cur, FwdRaw& spare) -> bool {
    const bool more = wn1.b < b1;
    FwdWin wn2 = wn1;
    if (more) {
      wn2 = next_win(wn1);
      terms(cur, wn1, buf[par ^ 1], spare, wn2, wn2.b < b1);
    }
    fold(buf[par], wc);
    if (!more || wn1.b != wc.b) {
      // Window k closes its block: combine, finalize, and take the next
      // block's rows.
      if (has) {
        const int u = pre.u;
        const float a = Mono<M>::op(d.acc ? d.acc[u] : ident, s);
        if (pre.fin) {
          run_program(d.apply, u, pre.f, a, 0.0f, true);
          if (d.acc) d.acc[u] = ident;
        } else if (d.acc) {
          d.acc[u] = a;
        }
      }
      s = ident;
      if (more) {
        fb = wn1.b;
        setup_rows();
      }
    }
    __syncthreads();
    if (!more) return true;
    wc = wn1;
    wn1 = wn2;
    par ^= 1;
    return false;
  };
  for (;;) {
    if (step(B, A)) break;
    if (step(A, B)) break;
  }
}

}  // namespace
