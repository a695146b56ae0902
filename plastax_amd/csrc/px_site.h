// px_site.h -- the site-program interpreter (growth, pruning and update
// callbacks traced to a small register machine), shared by the kernels that
// evaluate a program per site: the structural entry points and the forward
// pass that evaluates a PruneConn predicate in its sweep.
#pragma once

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

#include "../../include/plastax_hip.h"
#include "px_common.h"
#include "px_math.h"

namespace {

enum : int32_t {
  S_CONST = 1, S_IDX = 2, S_LDU = 3, S_LDC = 4, S_RNG = 5, S_MOV = 6, S_SEL = 7, S_OUT = 8,
  S_FADD = 10, S_FSUB, S_FMUL, S_FDIV, S_FNEG, S_FABS, S_FMAX, S_FMIN, S_FTANH, S_FEXP, S_FLOG,
  S_FSQRT, S_FSIGMOID, S_FSQUARE, S_FRELU, S_FSIGN, S_FFLOOR, S_FCOS, S_FSIN,
  S_FGT = 30, S_FGE, S_FLT, S_FLE, S_FEQ, S_FNE,
  S_IADD = 40, S_ISUB, S_IMUL, S_INEG, S_IABS, S_IMAX, S_IMIN, S_IFLOORDIV, S_IMOD, S_ISIGN,
  S_IGT = 50, S_IGE, S_ILT, S_ILE, S_IEQ, S_INE,
  S_UMAX = 60, S_UMIN, S_UFLOORDIV, S_UMOD, S_UGT, S_UGE, S_ULT, S_ULE,
  S_AND = 70, S_OR, S_XOR, S_NOT, S_SHL, S_SHRU, S_SHRI, S_BNOT,
  S_I2F = 80, S_U2F, S_F2I, S_F2U, S_F2B, S_I2B,
  S_FLOG1P = 90, S_FEXPM1 = 91
};

__device__ __forceinline__ float fmax_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}
__device__ __forceinline__ float fmin_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a < b ? a : b;
}
// Floor division and modulo of int32 (b == 0: -1 for a == 0 else -2, and a;
// INT32_MIN / -1 wraps).
__device__ __forceinline__ int32_t floordiv_i32(int32_t a, int32_t b) {
  if (b == 0) return a == 0 ? -1 : -2;
  if (a == INT32_MIN && b == -1) return INT32_MIN;
  int32_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) q -= 1;
  return q;
}
__device__ __forceinline__ int32_t mod_i32(int32_t a, int32_t b) {
  if (b == 0) return a;
  if (b == -1) return 0;
  int32_t r = a % b;
  if (r != 0 && ((r < 0) != (b < 0))) r += b;
  return r;
}
// The same values with selects only, for compiled programs: the divisor is
// often a program constant, uniform over the wave, and a branch on it would
// split the program into blocks the loads of the lane's next site cannot
// move above. (The interpreter keeps the branches: in its one big switch
// the selects' extra live values spill.)
__device__ __forceinline__ int32_t floordiv_i32_sel(int32_t a, int32_t b) {
  const bool zero = b == 0, wrap = a == INT32_MIN && b == -1;
  const int32_t bb = (zero || wrap) ? 1 : b;
  int32_t q = a / bb;
  const int32_t r = a - q * bb;  // the remainder, with a's sign (|q * bb| <= |a|)
  q -= (r != 0 && ((r < 0) != (bb < 0))) ? 1 : 0;
  return zero ? (a == 0 ? -1 : -2) : (wrap ? INT32_MIN : q);
}
__device__ __forceinline__ int32_t mod_i32_sel(int32_t a, int32_t b) {
  const int32_t bb = (b == 0 || b == -1) ? 1 : b;
  int32_t r = a % bb;
  r += (r != 0 && ((r < 0) != (bb < 0))) ? bb : 0;
  return b == 0 ? a : (b == -1 ? 0 : r);
}
__device__ __forceinline__ int32_t f2i(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return INT32_MAX;
  if (x <= -2147483648.0f) return INT32_MIN;
  return static_cast<int32_t>(x);
}
__device__ __forceinline__ uint32_t f2u(float x) {
  if (x != x || x <= 0.0f) return 0u;
  if (x >= 4294967296.0f) return UINT32_MAX;
  return static_cast<uint32_t>(x);
}
__device__ __forceinline__ uint32_t load32(const void* base, int32_t bytes, int64_t at) {
  if (bytes == 1) return static_cast<const uint8_t*>(base)[at] != 0;
  return static_cast<const uint32_t*>(base)[at];
}

struct Site {
  int32_t role[5];    // i, j, src, dst, cid (the position conn fields are read at)
  int32_t cid_value;  // the cid the program sees
  uint64_t seed;      // (keyed << 32) | key
  const int32_t* ids_logical;
  const int32_t* ids_physical;
  int32_t batch;      // unit columns are [num_units][batch] when > 1
  int32_t sample;     // the site's sample
};

// The interpreter's 32 registers. Every operand index comes from the
// program in the kernel arguments, so it is uniform across the wave; each
// access is a switch on it (a scalar branch) whose cases name one register,
// so the file stays in VGPRs instead of scratch memory.
struct SiteRegs {
  uint32_t r[32];
  __device__ __forceinline__ uint32_t get(int i) const {
    switch (i & 31) {
      case 0: return r[0];
      case 1: return r[1];
      case 2: return r[2];
      case 3: return r[3];
      case 4: return r[4];
      case 5: return r[5];
      case 6: return r[6];
      case 7: return r[7];
      case 8: return r[8];
      case 9: return r[9];
      case 10: return r[10];
      case 11: return r[11];
      case 12: return r[12];
      case 13: return r[13];
      case 14: return r[14];
      case 15: return r[15];
      case 16: return r[16];
      case 17: return r[17];
      case 18: return r[18];
      case 19: return r[19];
      case 20: return r[20];
      case 21: return r[21];
      case 22: return r[22];
      case 23: return r[23];
      case 24: return r[24];
      case 25: return r[25];
      case 26: return r[26];
      case 27: return r[27];
      case 28: return r[28];
      case 29: return r[29];
      case 30: return r[30];
      case 31: return r[31];
      default: return 0u;
    }
  }
  __device__ __forceinline__ void set(int i, uint32_t v) {
    switch (i & 31) {
      case 0: r[0] = v; return;
      case 1: r[1] = v; return;
      case 2: r[2] = v; return;
      case 3: r[3] = v; return;
      case 4: r[4] = v; return;
      case 5: r[5] = v; return;
      case 6: r[6] = v; return;
      case 7: r[7] = v; return;
      case 8: r[8] = v; return;
      case 9: r[9] = v; return;
      case 10: r[10] = v; return;
      case 11: r[11] = v; return;
      case 12: r[12] = v; return;
      case 13: r[13] = v; return;
      case 14: r[14] = v; return;
      case 15: r[15] = v; return;
      case 16: r[16] = v; return;
      case 17: r[17] = v; return;
      case 18: r[18] = v; return;
      case 19: r[19] = v; return;
      case 20: r[20] = v; return;
      case 21: r[21] = v; return;
      case 22: r[22] = v; return;
      case 23: r[23] = v; return;
      case 24: r[24] = v; return;
      case 25: r[25] = v; return;
      case 26: r[26] = v; return;
      case 27: r[27] = v; return;
      case 28: r[28] = v; return;
      case 29: r[29] = v; return;
      case 30: r[30] = v; return;
      case 31: r[31] = v; return;
      default: return;
    }
  }
};

static_assert(PLX_MAX_SOUTS == 8, "site_out names eight outputs");
__device__ __forceinline__ void site_out(uint32_t (&o)[PLX_MAX_SOUTS], int i, uint32_t v) {
  switch (i & 7) {
    case 0: o[0] = v; return;
    case 1: o[1] = v; return;
    case 2: o[2] = v; return;
    case 3: o[3] = v; return;
    case 4: o[4] = v; return;
    case 5: o[5] = v; return;
    case 6: o[6] = v; return;
    case 7: o[7] = v; return;
    default: return;
  }
}

// A launch's shape as the interpreter sees it: read from the descriptor,
// the site and the program at run time. A compiled program gets a shape
// whose answers are constants (the generated source's SiteShape), so its
// loads are straight-line code with no branch between them.
struct ShapeRT {
  static constexpr bool kSelects = false;  // integer division and modulo with branches
  __device__ __forceinline__ static int kind(const plx_site_desc& d) { return d.kind; }
  __device__ __forceinline__ static int32_t batch(const plx_site_desc& d) { return d.batch > 1 ? d.batch : 1; }
  __device__ __forceinline__ static bool from(const plx_site_desc& d) { return d.from_id != nullptr; }
  __device__ __forceinline__ static bool to(const plx_site_desc& d) { return d.to_id != nullptr; }
  __device__ __forceinline__ static bool site_ids(const plx_site_desc& d) { return d.site_ids != nullptr; }
  __device__ __forceinline__ static bool logical(const Site& c) { return c.ids_logical != nullptr; }
  __device__ __forceinline__ static bool physical(const Site& c) { return c.ids_physical != nullptr; }
  __device__ __forceinline__ static bool batched(const Site& c) { return c.batch > 1; }
  __device__ __forceinline__ static int32_t ubytes(const plx_site_prog& p, int a) { return p.ubytes[a]; }
  __device__ __forceinline__ static int32_t cbytes(const plx_site_prog& p, int a) { return p.cbytes[a]; }
};

// One instruction (op, d, a, b) of a site program. The interpreter calls it
// with the operands it reads from the program; a compiled program (the source
// plx_site_compile generates) calls it with literal operands, and the switch
// and the register selects fold away.
template <class Sh>
__device__ __forceinline__ void site_step(int op, int d, int a, int b, SiteRegs& r, const plx_site_prog& p,
                                          const Site& c, int32_t num_units, uint32_t (&outv)[PLX_MAX_SOUTS]) {
  {
    const uint32_t x = r.get(a), y = r.get(b);
    const int32_t xi = static_cast<int32_t>(x), yi = static_cast<int32_t>(y);
    const float xf = __uint_as_float(x), yf = __uint_as_float(y);
    uint32_t v = 0;
    switch (op) {
      case S_CONST: v = p.consts[a]; break;
      case S_IDX: {  // a is uniform: a switch keeps c.role in registers
        int32_t w = c.cid_value;
        switch (a) {
          case 0: w = c.role[0]; break;
          case 1: w = c.role[1]; break;
          case 2: w = c.role[2]; break;
          case 3: w = c.role[3]; break;
          default: break;
        }
        v = static_cast<uint32_t>(w);
        break;
      }
      case S_LDU: {
        int64_t at = yi;
        at = at < 0 ? 0 : (at > num_units - 1 ? num_units - 1 : at);
        if (Sh::physical(c)) at = c.ids_physical[at];
        if (Sh::batched(c)) at = at * c.batch + c.sample;
        v = load32(p.ufields[a], Sh::ubytes(p, a), at);
        break;
      }
      case S_LDC:
        v = load32(p.cfields[a], Sh::cbytes(p, a) & 0xFF, c.role[4]);
        if ((Sh::cbytes(p, a) & PLX_SITE_ID_COLUMN) && Sh::logical(c)) {
          const int32_t id = static_cast<int32_t>(v);
          v = static_cast<uint32_t>(c.ids_logical[id < 0 ? 0 : (id > num_units - 1 ? num_units - 1 : id)]);
        }
        break;
      case S_RNG:
        v = px::philox32(c.seed, (static_cast<uint64_t>(static_cast<uint32_t>(c.role[1])) << 16) |
                                     static_cast<uint32_t>(a));
        break;
      case S_MOV: v = x; break;
      case S_SEL: v = x ? r.get(b) : r.get(b + 1); break;
      case S_OUT: site_out(outv, d, x); return;
      case S_FADD: v = __float_as_uint(xf + yf); break;
      case S_FSUB: v = __float_as_uint(xf - yf); break;
      case S_FMUL: v = __float_as_uint(xf * yf); break;
      case S_FDIV: v = __float_as_uint(xf / yf); break;
      case S_FNEG: v = x ^ 0x80000000u; break;
      case S_FABS: v = x & 0x7FFFFFFFu; break;
      case S_FMAX: v = __float_as_uint(fmax_nan(xf, yf)); break;
      case S_FMIN: v = __float_as_uint(fmin_nan(xf, yf)); break;
      case S_FTANH: v = __float_as_uint(px::tanhf_(xf)); break;
      case S_FEXP: v = __float_as_uint(px::expf_(xf)); break;
      case S_FLOG: v = __float_as_uint(px::logf_(xf)); break;
      case S_FSQRT: v = __float_as_uint(__builtin_sqrtf(xf)); break;
      case S_FSIGMOID: v = __float_as_uint(px::sigmoidf_(xf)); break;
      case S_FCOS: v = __float_as_uint(px::cosf_(xf)); break;
      case S_FSIN: v = __float_as_uint(px::sinf_(xf)); break;
      case S_FLOG1P: v = __float_as_uint(px::log1pf_(xf)); break;
      case S_FEXPM1: v = __float_as_uint(px::expm1f_(xf)); break;
      case S_FSQUARE: v = __float_as_uint(xf * xf); break;
      case S_FRELU: v = __float_as_uint(fmax_nan(xf, 0.0f)); break;
      case S_FSIGN: v = xf > 0.0f ? 0x3F800000u : (xf < 0.0f ? 0xBF800000u : x); break;
      case S_FFLOOR: v = __float_as_uint(floorf(xf)); break;
      case S_FGT: v = xf > yf; break;
      case S_FGE: v = xf >= yf; break;
      case S_FLT: v = xf < yf; break;
      case S_FLE: v = xf <= yf; break;
      case S_FEQ: v = xf == yf; break;
      case S_FNE: v = xf != yf; break;
      case S_IADD: v = x + y; break;
      case S_ISUB: v = x - y; break;
      case S_IMUL: v = x * y; break;
      case S_INEG: v = 0u - x; break;
      case S_IABS: v = xi < 0 ? 0u - x : x; break;
      case S_IMAX: v = xi > yi ? x : y; break;
      case S_IMIN: v = xi < yi ? x : y; break;
      case S_IFLOORDIV:
        v = static_cast<uint32_t>(Sh::kSelects ? floordiv_i32_sel(xi, yi) : floordiv_i32(xi, yi));
        break;
      case S_IMOD: v = static_cast<uint32_t>(Sh::kSelects ? mod_i32_sel(xi, yi) : mod_i32(xi, yi)); break;
      case S_ISIGN: v = static_cast<uint32_t>(xi > 0 ? 1 : (xi < 0 ? -1 : 0)); break;
      case S_IGT: v = xi > yi; break;
      case S_IGE: v = xi >= yi; break;
      case S_ILT: v = xi < yi; break;
      case S_ILE: v = xi <= yi; break;
      case S_IEQ: v = x == y; break;
      case S_INE: v = x != y; break;
      case S_UMAX: v = x > y ? x : y; break;
      case S_UMIN: v = x < y ? x : y; break;
      case S_UFLOORDIV: v = y ? x / y : UINT32_MAX; break;
      case S_UMOD: v = y ? x % y : x; break;
      case S_UGT: v = x > y; break;
      case S_UGE: v = x >= y; break;
      case S_ULT: v = x < y; break;
      case S_ULE: v = x <= y; break;
      case S_AND: v = x & y; break;
      case S_OR: v = x | y; break;
      case S_XOR: v = x ^ y; break;
      case S_NOT: v = ~x; break;
      case S_BNOT: v = x == 0u; break;
      case S_SHL: v = y >= 32u ? 0u : x << y; break;
      case S_SHRU: v = y >= 32u ? 0u : x >> y; break;
      case S_SHRI: v = y >= 32u ? (xi < 0 ? UINT32_MAX : 0u) : static_cast<uint32_t>(xi >> y); break;
      case S_I2F: v = __float_as_uint(static_cast<float>(xi)); break;
      case S_U2F: v = __float_as_uint(static_cast<float>(x)); break;
      case S_F2I: v = static_cast<uint32_t>(f2i(xf)); break;
      case S_F2U: v = f2u(xf); break;
      case S_F2B: v = xf != 0.0f; break;
      case S_I2B: v = x != 0u; break;
      default: break;
    }
    r.set(d, v);
  }
}

// The interpreter: the program's instructions in order.
__device__ __forceinline__ void site_run(const plx_site_prog& p, const Site& c, int32_t num_units,
                                         uint32_t (&outv)[PLX_MAX_SOUTS]) {
  SiteRegs r;
  for (int k = 0; k < p.ninstr; ++k)
    site_step<ShapeRT>(p.code[4 * k], p.code[4 * k + 1], p.code[4 * k + 2], p.code[4 * k + 3], r, p, c, num_units,
                       outv);
}

struct SiteInterp {
  using Shape = ShapeRT;
  static constexpr int kSites = 1;  // sites per lane per pass of the kernel's loop
  __device__ __forceinline__ static void run(const plx_site_prog& p, const Site& c, int32_t num_units,
                                             uint32_t (&outv)[PLX_MAX_SOUTS]) {
    site_run(p, c, num_units, outv);
  }
};

__device__ __forceinline__ int64_t live_count(int64_t n_max, const int32_t* n_dev) {
  if (!n_dev) return n_max;
  const int64_t c = *n_dev;
  return c < n_max ? (c < 0 ? 0 : c) : n_max;
}

// plx_site_eval's sites (grid-strided): each site's roles and rng seed, the
// program (Prog::run: the interpreter, or a compiled program), then its
// outputs -- one column per output, or a kill ORed into or_into. Each lane
// takes Prog::kSites sites per pass (a stride apart): their programs run
// before any output is stored, so a compiled program's loads for all of them
// are in flight together.
template <class Sh>
__device__ __forceinline__ void site_setup(const plx_site_desc& d, int64_t s, int64_t per, uint32_t keyed, Site& c) {
  c.role[0] = c.role[1] = c.role[2] = c.role[3] = c.role[4] = 0;
  uint32_t key = 0;
  c.batch = Sh::batch(d);
  c.sample = d.sample;
  c.ids_logical = d.ids_logical;
  c.ids_physical = d.ids_physical;
  switch (Sh::kind(d)) {
    case PLX_SITES_UNIT:
      if (c.batch > 1) {  // (unit, sample) sites over [num_units][batch] columns
        c.role[0] = static_cast<int32_t>(s / c.batch);
        c.sample = static_cast<int32_t>(s % c.batch);
        key = static_cast<uint32_t>(c.role[0]);
        break;
      }
      c.role[0] = static_cast<int32_t>(s / per);
      c.role[1] = static_cast<int32_t>(s % per);
      key = static_cast<uint32_t>(c.role[0]);
      break;
    case PLX_SITES_GLOBAL: c.role[1] = static_cast<int32_t>(s); break;
    case PLX_SITES_CONN: {
      const int32_t cid = d.list_a[s / per];
      c.role[1] = static_cast<int32_t>(s % per);
      c.role[2] = d.from_id[cid];
      c.role[3] = d.to_id[cid];
      c.role[4] = cid;
      const uint64_t pair = (static_cast<uint64_t>(static_cast<uint32_t>(c.role[2])) << 32) |
                            static_cast<uint32_t>(c.role[3]);
      key = px::philox32(pair, static_cast<uint32_t>(d.occ[cid]));
      break;
    }
    case PLX_SITES_GRID: {
      const int64_t m2 = per * per;
      const int64_t g = s / m2, rem = s - g * m2;
      c.role[2] = d.list_a[g * per + rem / per];
      c.role[3] = d.list_b[g * per + rem % per];
      break;
    }
    case PLX_SITES_PAIRS:
      c.role[2] = d.list_a[s];
      c.role[3] = d.list_b[s];
      break;
    default: {  // EDGE: the edge's own slot; its endpoints when the ids are passed
      c.role[4] = static_cast<int32_t>(s);
      const int32_t* lg = d.ids_logical;
      if (Sh::from(d)) c.role[2] = Sh::logical(c) ? lg[d.from_id[s]] : d.from_id[s];
      if (Sh::to(d)) c.role[3] = Sh::logical(c) ? lg[d.to_id[s]] : d.to_id[s];
      break;
    }
  }
  c.cid_value = c.role[4];
  if (Sh::site_ids(d)) {
    if (Sh::kind(d) == PLX_SITES_EDGE) c.cid_value = d.site_ids[s];
    if (Sh::kind(d) == PLX_SITES_UNIT) c.role[0] = d.site_ids[c.batch > 1 ? s / c.batch : s / per];
  }
  c.seed = (static_cast<uint64_t>(keyed) << 32) | key;
}

// Lanes per workgroup of every site-program launch (a constant, so the
// kernel reads no launch size from memory).
constexpr int kSiteBlock = 256;

template <class Prog>
__device__ __forceinline__ void site_eval_body(const plx_site_desc& d) {
  constexpr int K = Prog::kSites;
  const int64_t n = live_count(d.n, d.n_dev);
  const uint32_t keyed =
      px::philox32(d.net_seed, (static_cast<uint64_t>(static_cast<uint32_t>(d.step)) << 8) | 1u);
  const int64_t per = d.per > 0 ? d.per : 1;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kSiteBlock;
  for (int64_t s0 = static_cast<int64_t>(blockIdx.x) * kSiteBlock + threadIdx.x; s0 < n; s0 += K * stride) {
    uint32_t out[K][PLX_MAX_SOUTS];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      // A site past the end evaluates the last site again (s0 < n) and
      // stores nothing: no branch around the program, so the loads of the
      // lane's sites can all be issued before the first is used.
      const int64_t s = K > 1 ? min(s0 + k * stride, n - 1) : s0;
      Site c;
      site_setup<typename Prog::Shape>(d, s, per, keyed, c);
      Prog::run(d.prog, c, d.num_units, out[k]);
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int64_t s = s0 + k * stride;
      if (s >= n) continue;
      if (d.or_into) {
        if (out[k][0] && !d.or_into[s]) {
          d.or_into[s] = 1;
          if (d.stamp) d.stamp[s] = d.stamp_value;
          if (d.kill_count) atomicAdd(d.kill_count, 1);
        }
      } else {
#pragma unroll
        for (int j = 0; j < PLX_MAX_SOUTS; ++j)
          if (j < d.prog.nout) static_cast<uint32_t*>(d.outs[j])[s] = out[k][j];
      }
    }
  }
}

}  // namespace
