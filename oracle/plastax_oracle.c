/*
 * plastax_oracle.c -- CPU restatement of the reference's streaming-step
 * arithmetic. TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, always as the checker, never as
 * the thing measured or shipped. The product path (plastax_amd) never links
 * or calls anything in this directory.
 *
 * Every function below restates one piece of the reference (Sir-NoChill/
 * plastax, src/plastax/...) and cites the lines it follows. The level walks
 * and phase order live in oracle.py (which mirrors phases.py); this file
 * holds the O(E) loops.
 *
 * Summation order. The reference's per-bucket reduction is XLA's scatter
 * (jax.ops.segment_sum, monoid.py:84-122), which on the CPU folds updates in
 * slot order into a zero-filled output. The forward fold here is exactly
 * that. The backward fold (ox_bucket_reduce_bwd_tiled) follows each source's
 * terms in destination-sorted order, grouped by the device's fixed tiles of
 * that order: each tile's terms are folded from the identity and the tile sums
 * are folded in order (the deterministic tree of the device's transpose
 * reduce). ox_bucket_reduce_bwd keeps the plain slot-order fold (optionally in
 * pieces) for comparisons against the reference's literal order.
 *
 * Build: see Makefile (gcc -O3 -ffp-contract=off: no contraction, so every
 * product and sum rounds to float32 exactly as the reference's jnp ops do).
 * Built with -DOX_LIBM_ELEMENTARY (libplastax_oracle_libm.so), exp, log and
 * tanh come from the C library instead: that build only serves the
 * perturbation study of oracle/perturb.py and is never a parity oracle.
 * The per-edge and per-unit loops run under OpenMP when it is on: every
 * iteration writes its own slot and every fold keeps its order inside one
 * iteration, so the results do not depend on the thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OX_API __attribute__((visibility("default")))

#ifdef _OPENMP
#include <omp.h>
#endif

/* Loops of at least this many iterations run on the OpenMP team. */
#define OX_PAR_MIN 65536

/* The OpenMP team size for later calls (1: sequential); returns the size
 * in force, 1 when built without OpenMP. */
OX_API int32_t ox_set_threads(int32_t n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
  return omp_get_max_threads();
#else
  (void)n;
  return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Philox-4x32-10: rng.py:109-141, scripts/parity/reference.py:153-184.      */
/* The core takes a general 4-word counter and 2-word key so it can be       */
/* pinned to the Random123 known-answer vectors; the plastax mapping loads   */
/* the block as (ctr_lo, ctr_hi, seed_lo, seed_hi), key (seed_lo, seed_hi).  */
/* ------------------------------------------------------------------------ */

OX_API void ox_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2],
                             uint32_t out[4]) {
  uint32_t x0 = ctr[0], x1 = ctr[1], x2 = ctr[2], x3 = ctr[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)0xD2511F53u * x0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * x2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ x1 ^ k0;
    uint32_t n2 = hi0 ^ x3 ^ k1;
    x0 = n0;
    x1 = lo1;
    x2 = n2;
    x3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = x0;
  out[1] = x1;
  out[2] = x2;
  out[3] = x3;
}

OX_API uint32_t ox_philox32(uint64_t seed, uint64_t counter) {
  uint32_t ctr[4] = {(uint32_t)counter, (uint32_t)(counter >> 32),
                     (uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t out[4];
  ox_philox4x32_10(ctr, key, out);
  return out[0];
}

OX_API void ox_philox32_batch(const uint64_t* seeds, const uint64_t* ctrs,
                              uint32_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = ox_philox32(seeds[i], ctrs[i]);
}

/* unit_float: rng.py:144-153 -- float32(word >> 8) * 2^-24. */
OX_API float ox_unit_float(uint32_t word) {
  return (float)(word >> 8) * (1.0f / 16777216.0f);
}

/* Rng.for_site: rng.py:206-246 -- (philox(net_seed, (step<<8)|stream) << 32) | key. */
OX_API uint64_t ox_site_seed(uint64_t net_seed, uint32_t step, uint32_t stream,
                             uint32_t key) {
  uint64_t ctr = ((uint64_t)step << 8) | (uint64_t)(stream & 0xFFu);
  uint64_t hi = ox_philox32(net_seed, ctr);
  return (hi << 32) | (uint64_t)key;
}

/* conn_key: rng.py:156-180 -- philox((src << 32) | dst, occurrence). */
OX_API uint32_t ox_conn_key(uint32_t src, uint32_t dst, uint32_t occ) {
  return ox_philox32(((uint64_t)src << 32) | (uint64_t)dst, (uint64_t)occ);
}

/* Rng._draw: rng.py:248-259 -- philox(site_seed, (j << 16) | sub). */
OX_API uint32_t ox_site_draw(uint64_t site_seed, uint32_t j, uint32_t sub) {
  return ox_philox32(site_seed, ((uint64_t)j << 16) | (uint64_t)(sub & 0xFFFFu));
}

/* Rng.uniform_int: rng.py:273-287 -- min(uint32(u * n), n - 1). */
OX_API uint32_t ox_uniform_int(uint32_t word, uint32_t n) {
  float u = ox_unit_float(word);
  float s = u * (float)n;
  uint32_t k = (uint32_t)s;
  return k < n - 1u ? k : n - 1u;
}

/* ------------------------------------------------------------------------ */
/* Elementary functions. The reference evaluates jnp.exp/tanh/log with       */
/* XLA's own approximations, which cannot be reproduced bit for bit here.    */
/* The framework defines them by the Cephes single-precision algorithms      */
/* (S. L. Moshier, Cephes Math Library: expf.c, logf.c, tanhf.c), written    */
/* with plain float32 +,-,*,/ only, so a CPU build with contraction off and   */
/* the device build give identical bits. Accuracy: <= 2 ulp against the      */
/* double-precision libm (pinned in tests/test_oracle_math.py).              */
/* ------------------------------------------------------------------------ */

static inline float ox_bits_to_float(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}
static inline uint32_t ox_float_to_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}
/* 2^n as a float32, n in [-126, 127]. */
static inline float ox_pow2i(int n) {
  return ox_bits_to_float((uint32_t)(n + 127) << 23);
}

OX_API float ox_expf(float x) {
#ifdef OX_LIBM_ELEMENTARY
  return expf(x); /* perturbation build (oracle/perturb.py) */
#endif
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.97208404541015625f) return 0.0f;
  float fn = floorf(x * 1.44269502162933349609375f + 0.5f);
  int n = (int)fn;
  float r = x - fn * 0.693359375f;
  r = r - fn * -2.12194440e-4f;
  float z = r * r;
  float p = 1.9875691500e-4f;
  p = p * r + 1.3981999507e-3f;
  p = p * r + 8.3334519073e-3f;
  p = p * r + 4.1665795894e-2f;
  p = p * r + 1.6666665459e-1f;
  p = p * r + 5.0000001201e-1f;
  p = p * z + r;
  p = p + 1.0f;
  if (n > 127) return (p * ox_pow2i(127)) * ox_pow2i(n - 127);
  if (n < -126) return (p * ox_pow2i(n + 64)) * ox_pow2i(-64);
  return p * ox_pow2i(n);
}

OX_API float ox_logf(float x) {
#ifdef OX_LIBM_ELEMENTARY
  return logf(x); /* perturbation build (oracle/perturb.py) */
#endif
  if (x != x) return x;
  if (x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (x == INFINITY) return x;
  int e = 0;
  uint32_t b = ox_float_to_bits(x);
  if ((b >> 23) == 0) { /* subnormal: scale into the normal range */
    x = x * 33554432.0f; /* 2^25 */
    b = ox_float_to_bits(x);
    e = -25;
  }
  e += (int)((b >> 23) & 0xFFu) - 126;
  float m = ox_bits_to_float((b & 0x007FFFFFu) | 0x3F000000u); /* [0.5, 1) */
  if (m < 0.707106781186547524f) {
    e -= 1;
    m = m + m - 1.0f;
  } else {
    m = m - 1.0f;
  }
  float z = m * m;
  float y = 7.0376836292e-2f;
  y = y * m - 1.1514610310e-1f;
  y = y * m + 1.1676998740e-1f;
  y = y * m - 1.2420140846e-1f;
  y = y * m + 1.4249322787e-1f;
  y = y * m - 1.6668057665e-1f;
  y = y * m + 2.0000714765e-1f;
  y = y * m - 2.4999993993e-1f;
  y = y * m + 3.3333331174e-1f;
  y = y * m;
  y = y * z;
  float fe = (float)e;
  if (e != 0) y = y + -2.12194440e-4f * fe;
  y = y + -0.5f * z;
  float r = m + y;
  if (e != 0) r = r + 0.693359375f * fe;
  return r;
}

OX_API float ox_tanhf(float x) {
#ifdef OX_LIBM_ELEMENTARY
  return tanhf(x); /* perturbation build (oracle/perturb.py) */
#endif
  float z = fabsf(x);
  if (z > 44.36141967773437500f) return x > 0.0f ? 1.0f : -1.0f;
  if (z >= 0.625f) {
    float s = ox_expf(z + z);
    float t = 1.0f - 2.0f / (s + 1.0f);
    return x < 0.0f ? -t : t;
  }
  if (x == 0.0f) return x;
  float y = x * x;
  float p = -5.70498872745e-3f;
  p = p * y + 2.06390887954e-2f;
  p = p * y - 5.37397155531e-2f;
  p = p * y + 1.33314422036e-1f;
  p = p * y - 3.33332819422e-1f;
  p = p * y;
  p = p * x;
  return p + x;
}

OX_API float ox_sigmoidf(float x) { return 1.0f / (1.0f + ox_expf(-x)); }

/* log1p and expm1 by Kahan's method (Goldberg, "What Every Computer
 * Scientist Should Know About Floating-Point Arithmetic", 1991, Theorem 4):
 * u = fl(1 + x), log1p = x * (log(u) / (u - 1)); u = exp(x),
 * expm1 = (u - 1) * (x / log(u)); exact where u == 1, infinities pass. */
OX_API float ox_log1pf(float x) {
  const float u = 1.0f + x;
  if (u == 1.0f) return x;
  if (u == INFINITY) return u;
  return x * (ox_logf(u) / (u - 1.0f));
}

OX_API float ox_expm1f(float x) {
  const float u = ox_expf(x);
  if (u == 1.0f) return x;
  if (u == INFINITY) return u;
  const float um1 = u - 1.0f;
  if (um1 == -1.0f) return -1.0f;
  return um1 * (x / ox_logf(u));
}

/* sin and cos follow Cephes sinf.c / cosf.c (Moshier): |x| is reduced */
/* modulo pi/4 by the octant j = trunc(|x| * 4/pi), rounded up to even, and */
/* r = |x| - j * pi/4 with pi/4 split in three (DP1 and DP2 have few */
/* significant bits, so j * DP1 and j * DP2 are exact while |x| <= 8192); */
/* the sine or cosine minimax polynomial of r on [-pi/4, pi/4] is chosen by */
/* octant. Past 8192 the reduction loses precision (Cephes' PLOSS), past */
/* 2^24 - 1 the result is 0 (TLOSS); infinities and NaN give NaN. */
static float ox_sincos_reduce(float x, int j) {
  if (x > 8192.0f)
    x = x - (float)j * 0.7853981633974483096f;
  else
    x = ((x - (float)j * 0.78515625f) - (float)j * 2.4187564849853515625e-4f) -
        (float)j * 3.77489497744594108e-8f;
  return x;
}

static float ox_sin_poly(float x, float z) {
  float r = ((-1.9515295891e-4f * z + 8.3321608736e-3f) * z - 1.6666654611e-1f) * z * x;
  return r + x;
}

static float ox_cos_poly(float z) {
  float r = ((2.443315711809948e-5f * z - 1.388731625493765e-3f) * z + 4.166664568298827e-2f) * z * z;
  r = r - 0.5f * z;
  return r + 1.0f;
}

OX_API float ox_cosf(float xx) {
  if (xx != xx) return xx;
  const float x = fabsf(xx);
  if (x == INFINITY) return NAN;
  if (x > 16777215.0f) return 0.0f;
  int j = (int)(1.27323954473516f * x);
  int y = j;
  if (j & 1) {
    j += 1;
    y += 1;
  }
  j &= 7;
  int neg = 0;
  if (j > 3) {
    j -= 4;
    neg = 1;
  }
  if (j > 1) neg = !neg;
  const float r = ox_sincos_reduce(x, y);
  const float z = r * r;
  const float v = (j == 1 || j == 2) ? ox_sin_poly(r, z) : ox_cos_poly(z);
  return neg ? -v : v;
}

OX_API float ox_sinf(float xx) {
  if (xx != xx) return xx;
  int neg = signbit(xx) != 0; /* sin(-0) = -0 */
  const float x = fabsf(xx);
  if (x == INFINITY) return NAN;
  if (x > 16777215.0f) return 0.0f;
  int j = (int)(1.27323954473516f * x);
  int y = j;
  if (j & 1) {
    j += 1;
    y += 1;
  }
  j &= 7;
  if (j > 3) {
    neg = !neg;
    j -= 4;
  }
  const float r = ox_sincos_reduce(x, y);
  const float z = r * r;
  const float v = (j == 1 || j == 2) ? ox_cos_poly(z) : ox_sin_poly(r, z);
  return neg ? -v : v;
}


/* NaN-propagating max/min, as jnp.maximum / jnp.minimum (monoid.py:46-51). */
static inline float ox_fmax_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}
static inline float ox_fmin_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a < b ? a : b;
}

/* b^t for the Adam bias correction (_adam.py:164-165 computes
 * float32(b) ** float32(t)). For an integer-valued t in [0, 2^24] the power
 * is taken by binary exponentiation in float64 and rounded once to float32
 * (every double product is correctly rounded, so the device reproduces the
 * bits); any other t goes through powf. */
OX_API float ox_pow_step(float b, float t) {
  if (t >= 0.0f && t <= 16777216.0f && floorf(t) == t) {
    uint32_t n = (uint32_t)t;
    double base = (double)b, acc = 1.0;
    while (n) {
      if (n & 1u) acc *= base;
      base *= base;
      n >>= 1;
    }
    return (float)acc;
  }
  return powf(b, t);
}

/* ------------------------------------------------------------------------ */
/* Monoid segment reduce of one bucket (sweep.py:113-180, monoid.py:84-122). */
/* ------------------------------------------------------------------------ */

enum { OX_SUM = 0, OX_PROD = 1, OX_MAX = 2, OX_MIN = 3 };

static inline float ox_combine1(int monoid, float a, float b) {
  switch (monoid) {
    case OX_SUM: return a + b;
    case OX_PROD: return a * b;
    case OX_MAX: return ox_fmax_nan(a, b);
    default: return ox_fmin_nan(a, b);
  }
}

OX_API float ox_identity(int monoid) {
  switch (monoid) {
    case OX_SUM: return 0.0f;
    case OX_PROD: return 1.0f;
    case OX_MAX: return -INFINITY;
    default: return INFINITY;
  }
}

/* Forward accumulate of one bucket: out[t] (pre-filled with the identity)
 * folds map(e) = weight[e] * x[from[e]] over the live slots targeting t, in
 * slot order (the null-slot trick of sweep.py:158-161 drops dead slots). */
OX_API void ox_bucket_reduce_fwd(int64_t cap, const int32_t* from,
                                 const int32_t* to, const uint8_t* dead,
                                 const float* weight, const float* x,
                                 int32_t monoid, float* out) {
  for (int64_t e = 0; e < cap; ++e) {
    if (dead[e]) continue;
    float v = weight[e] * x[from[e]];
    out[to[e]] = ox_combine1(monoid, out[to[e]], v);
  }
}

/* Backward accumulate of one bucket into FROM_ID (sweep.py:371-399 with
 * target=FROM_ID): map(e) = weight[e] * g[to[e]], folded per source in slot
 * order, in pieces of at most `piece` terms (see the header). `pc`/`pn` are
 * caller scratch of num_units floats / ints, zeroed here. */
OX_API void ox_bucket_reduce_bwd(int64_t cap, const int32_t* from,
                                 const int32_t* to, const uint8_t* dead,
                                 const float* weight, const float* g,
                                 int32_t num_units, int32_t monoid,
                                 int32_t piece, float* out, float* pc,
                                 int32_t* pn) {
  float id = ox_identity(monoid);
  for (int32_t i = 0; i < num_units; ++i) {
    pc[i] = id;
    pn[i] = 0;
  }
  /* out[s] is the running fold of completed piece sums, pre-filled by the
   * caller with the identity (the fresh segment_reduce output). */
  for (int64_t e = 0; e < cap; ++e) {
    if (dead[e]) continue;
    int32_t s = from[e];
    float v = weight[e] * g[to[e]];
    pc[s] = ox_combine1(monoid, pc[s], v);
    if (++pn[s] == piece) {
      out[s] = ox_combine1(monoid, out[s], pc[s]);
      pc[s] = id;
      pn[s] = 0;
    }
  }
  for (int32_t s = 0; s < num_units; ++s)
    if (pn[s]) out[s] = ox_combine1(monoid, out[s], pc[s]);
}

/* Backward accumulate of one bucket in the device's tiled order. `order`
 * lists the bucket's n live slots sorted by (src, dst, slot) -- for each
 * source, its terms in the physical (destination-sorted) order -- and
 * tile[e] / sb[e] are slot e's tile and superblock (both non-decreasing in
 * that physical order). Per source, the terms of each tile are folded from
 * the identity in order; the tile sums of each superblock are folded in tile
 * order; the superblock sums are folded in order into out[s] (pre-filled
 * with the identity). With one tile this is the plain fold of each source's
 * terms in (dst, slot) order, which is the slot order of a source-major
 * bucket (builder.py:566-579). */
OX_API void ox_bucket_reduce_bwd_tiled(int64_t n, const int64_t* order,
                                       const int32_t* from, const int32_t* to,
                                       const float* weight, const float* g,
                                       const int32_t* tile, const int32_t* sb,
                                       int32_t monoid, float* out) {
  float id = ox_identity(monoid);
  int64_t k = 0;
  while (k < n) {
    int32_t s = from[order[k]];
    float total = out[s];
    while (k < n && from[order[k]] == s) {
      int32_t b = sb[order[k]];
      float sbsum = id;
      while (k < n && from[order[k]] == s && sb[order[k]] == b) {
        int32_t t = tile[order[k]];
        float part = id;
        while (k < n && from[order[k]] == s && tile[order[k]] == t) {
          int64_t e = order[k];
          part = ox_combine1(monoid, part, weight[e] * g[to[e]]);
          ++k;
        }
        sbsum = ox_combine1(monoid, sbsum, part);
      }
      total = ox_combine1(monoid, total, sbsum);
    }
    out[s] = total;
  }
}

/* ox_bucket_reduce_fwd by destination rows: row r folds, into
 * out[row_unit[r]] (pre-filled with the identity), the terms of the live
 * slots row_slots[row_ptr[r] .. row_ptr[r+1]) -- that destination's live
 * slots in ascending slot order -- so every destination sees the same fold
 * as the slot-order loop, and the rows run in parallel. */
OX_API void ox_bucket_reduce_fwd_rows(int64_t nrows, const int64_t* row_ptr,
                                      const int64_t* row_slots,
                                      const int32_t* row_unit,
                                      const int32_t* from, const float* weight,
                                      const float* x, int32_t monoid,
                                      float* out) {
#pragma omp parallel for schedule(dynamic, 256) if (nrows >= 1024)
  for (int64_t r = 0; r < nrows; ++r) {
    float v = out[row_unit[r]];
    for (int64_t k = row_ptr[r]; k < row_ptr[r + 1]; ++k) {
      int64_t e = row_slots[k];
      v = ox_combine1(monoid, v, weight[e] * x[from[e]]);
    }
    out[row_unit[r]] = v;
  }
}

/* ox_bucket_reduce_bwd_tiled by source runs: `order` as there, cut into
 * nruns runs of one source each (run_off[k] .. run_off[k+1]); each run is
 * that source's whole fold, so the runs are independent and run in
 * parallel. */
OX_API void ox_bucket_reduce_bwd_tiled_runs(int64_t nruns, const int64_t* run_off,
                                            const int64_t* order,
                                            const int32_t* from, const int32_t* to,
                                            const float* weight, const float* g,
                                            const int32_t* tile, const int32_t* sb,
                                            int32_t monoid, float* out) {
  float id = ox_identity(monoid);
#pragma omp parallel for schedule(dynamic, 256) if (nruns >= 1024)
  for (int64_t q = 0; q < nruns; ++q) {
    int64_t k = run_off[q];
    const int64_t end = run_off[q + 1];
    if (k >= end) continue;
    int32_t s = from[order[k]];
    float total = out[s];
    while (k < end) {
      int32_t b = sb[order[k]];
      float sbsum = id;
      while (k < end && sb[order[k]] == b) {
        int32_t t = tile[order[k]];
        float part = id;
        while (k < end && tile[order[k]] == t) {
          int64_t e = order[k];
          part = ox_combine1(monoid, part, weight[e] * g[to[e]]);
          ++k;
        }
        sbsum = ox_combine1(monoid, sbsum, part);
      }
      total = ox_combine1(monoid, total, sbsum);
    }
    out[s] = total;
  }
}

/* combine_pairwise (monoid.py:124-152): acc = acc op b, elementwise. */
OX_API void ox_combine(int64_t n, int32_t monoid, float* acc, const float* b) {
#pragma omp parallel for schedule(static) if (n >= OX_PAR_MIN)
  for (int64_t i = 0; i < n; ++i) acc[i] = ox_combine1(monoid, acc[i], b[i]);
}

/* ------------------------------------------------------------------------ */
/* Unit programs: a user Apply (sweep.py:183-230) or per-output loss term,    */
/* traced by the framework into a register program. Opcodes mirror           */
/* plastax_amd/_expr.py. Each instruction is 4 int32: op, dst, a, b.          */
/* ------------------------------------------------------------------------ */

enum {
  OP_ACC = 1,   /* r[d] = acc                         */
  OP_LDU = 2,   /* r[d] = field[a][i]                 */
  OP_CONST = 3, /* r[d] = consts[a]                   */
  OP_ADD = 4,
  OP_SUB = 5,
  OP_MUL = 6,
  OP_DIV = 7,
  OP_NEG = 8,
  OP_ABS = 9,
  OP_MAX = 10,
  OP_MIN = 11,
  OP_TANH = 12,
  OP_EXP = 13,
  OP_LOG = 14,
  OP_SQRT = 15,
  OP_SIGMOID = 16,
  OP_GT = 17,
  OP_GE = 18,
  OP_LT = 19,
  OP_LE = 20,
  OP_EQ = 21,
  OP_NE = 22,
  OP_SEL = 23,  /* r[d] = r[a] != 0 ? r[b] : r[b+1]   */
  OP_OUT = 24,  /* out slot d <- r[a]                 */
  OP_LDX = 25,  /* r[d] = aux0[k] (e.g. the target)   */
  OP_MOV = 26,
  OP_SQUARE = 27,
  OP_RELU = 28,
  OP_SIGN = 29,
  OP_LOG1P = 30,
  OP_EXPM1 = 31,
  OP_POW = 32,
  OP_COS = 33,
  OP_SIN = 34
};

#define OX_NREG 32
#define OX_NOUT 8

static float ox_run_program(const int32_t* prog, int32_t ninstr,
                            const float* consts, float* const* fields,
                            int64_t i, float acc, const float* aux0, int64_t k_aux,
                            float* outs) {
  float r[OX_NREG];
  for (int32_t k = 0; k < ninstr; ++k) {
    const int32_t* q = prog + 4 * k;
    int32_t d = q[1], a = q[2], b = q[3];
    switch (q[0]) {
      case OP_ACC: r[d] = acc; break;
      case OP_LDU: r[d] = fields[a][i]; break;
      case OP_CONST: r[d] = consts[a]; break;
      case OP_LDX: r[d] = aux0[k_aux]; break;
      case OP_MOV: r[d] = r[a]; break;
      case OP_ADD: r[d] = r[a] + r[b]; break;
      case OP_SUB: r[d] = r[a] - r[b]; break;
      case OP_MUL: r[d] = r[a] * r[b]; break;
      case OP_DIV: r[d] = r[a] / r[b]; break;
      case OP_NEG: r[d] = -r[a]; break;
      case OP_ABS: r[d] = fabsf(r[a]); break;
      case OP_SQUARE: r[d] = r[a] * r[a]; break;
      case OP_MAX: r[d] = ox_fmax_nan(r[a], r[b]); break;
      case OP_MIN: r[d] = ox_fmin_nan(r[a], r[b]); break;
      case OP_RELU: r[d] = ox_fmax_nan(r[a], 0.0f); break;
      case OP_TANH: r[d] = ox_tanhf(r[a]); break;
      case OP_EXP: r[d] = ox_expf(r[a]); break;
      case OP_LOG: r[d] = ox_logf(r[a]); break;
      case OP_SQRT: r[d] = sqrtf(r[a]); break;
      case OP_SIGMOID: r[d] = ox_sigmoidf(r[a]); break;
      case OP_COS: r[d] = ox_cosf(r[a]); break;
      case OP_SIN: r[d] = ox_sinf(r[a]); break;
      case OP_LOG1P: r[d] = ox_log1pf(r[a]); break;
      case OP_EXPM1: r[d] = ox_expm1f(r[a]); break;
      case OP_SIGN:
        r[d] = r[a] > 0.0f ? 1.0f : (r[a] < 0.0f ? -1.0f : r[a]);
        break;
      case OP_GT: r[d] = r[a] > r[b] ? 1.0f : 0.0f; break;
      case OP_GE: r[d] = r[a] >= r[b] ? 1.0f : 0.0f; break;
      case OP_LT: r[d] = r[a] < r[b] ? 1.0f : 0.0f; break;
      case OP_LE: r[d] = r[a] <= r[b] ? 1.0f : 0.0f; break;
      case OP_EQ: r[d] = r[a] == r[b] ? 1.0f : 0.0f; break;
      case OP_NE: r[d] = r[a] != r[b] ? 1.0f : 0.0f; break;
      case OP_SEL: r[d] = r[a] != 0.0f ? r[b] : r[b + 1]; break;
      case OP_OUT: outs[d] = r[a]; break;
      default: return NAN;
    }
  }
  return r[0];
}

/* Masked apply over every unit slot (sweep.py:183-230): writes out slot k of
 * the program into fields[out_field[k]] where mask[i], and resets acc there
 * to the identity. Every unit is evaluated against the pre-apply columns. */
OX_API void ox_apply(const int32_t* prog, int32_t ninstr, const float* consts,
                     float* const* fields, const int32_t* out_field,
                     int32_t nout, int64_t num_units, float* acc,
                     const uint8_t* mask, int32_t monoid, float* scratch) {
#pragma omp parallel for schedule(static) if (num_units >= OX_PAR_MIN)
  for (int64_t i = 0; i < num_units; ++i) {
    float outs[OX_NOUT];
    if (!mask[i]) continue;
    ox_run_program(prog, ninstr, consts, fields, i, acc[i], NULL, 0, outs);
    for (int32_t k = 0; k < nout; ++k) scratch[k * num_units + i] = outs[k];
  }
  float id = ox_identity(monoid);
#pragma omp parallel for schedule(static) if (num_units >= OX_PAR_MIN)
  for (int64_t i = 0; i < num_units; ++i) {
    if (!mask[i]) continue;
    for (int32_t k = 0; k < nout; ++k)
      fields[out_field[k]][i] = scratch[k * num_units + i];
    acc[i] = id;
  }
}

/* Piecewise fold of n terms: consecutive pieces of `piece` terms are each
 * folded from +0.0 in order, then the piece sums are folded in order. With
 * n <= piece this is the plain left-to-right float32 sum of the reference's
 * loss (scripts/parity/reference.py mse_loss_grad). */
static float ox_fold_pieces(const float* terms, int64_t n, int32_t piece) {
  float total = 0.0f;
  for (int64_t p0 = 0; p0 < n; p0 += piece) {
    float s = 0.0f;
    int64_t end = p0 + piece < n ? p0 + piece : n;
    for (int64_t k = p0; k < end; ++k) s = s + terms[k];
    total = total + s;
  }
  return total;
}

/* Elementwise loss (phases.py:1107-1131 with an elementwise policy such as
 * the reference's MSELoss): for output k, the program (prediction fields at
 * the output's unit, target at k) yields out slot 0 = seed and out slot 1 =
 * the loss term; the loss is the piecewise fold of the terms. `terms` is
 * caller scratch of n_out floats. */
OX_API float ox_loss_elementwise(const int32_t* prog, int32_t ninstr,
                                 const float* consts, float* const* fields,
                                 const int32_t* output_ids, int32_t n_out,
                                 const float* targets, float* seed_out,
                                 float* terms, int32_t piece) {
  float outs[OX_NOUT];
  for (int32_t k = 0; k < n_out; ++k) {
    ox_run_program(prog, ninstr, consts, fields, output_ids[k], 0.0f, targets,
                   k, outs);
    seed_out[k] = outs[0];
    terms[k] = outs[1];
  }
  return 0.0f + ox_fold_pieces(terms, n_out, piece);
}

/* SoftmaxCrossEntropyLoss (traits.py:204-250; op order of
 * scripts/parity/reference.py softmax_ce_loss_grad): running '>' max from
 * -inf, the piecewise sum of exp(a - m) in output order, then per output
 * seed = exp(z) / s - t and loss = piecewise fold of t * (log(s) - z).
 * `terms` is caller scratch of n_out floats. */
OX_API float ox_loss_softmax_ce(const float* act, const int32_t* output_ids,
                                int32_t n_out, const float* targets,
                                float* seed_out, float* terms, int32_t piece) {
  float peak = -INFINITY;
  for (int32_t k = 0; k < n_out; ++k) {
    float a = act[output_ids[k]];
    if (a > peak) peak = a;
  }
  for (int32_t k = 0; k < n_out; ++k) terms[k] = ox_expf(act[output_ids[k]] - peak);
  float total_exp = ox_fold_pieces(terms, n_out, piece);
  float log_sum = ox_logf(total_exp);
  for (int32_t k = 0; k < n_out; ++k) {
    float z = act[output_ids[k]] - peak;
    float t = targets[k];
    seed_out[k] = ox_expf(z) / total_exp - t;
    terms[k] = t * (log_sum - z);
  }
  return 0.0f + ox_fold_pieces(terms, n_out, piece);
}

/* ------------------------------------------------------------------------ */
/* Connection updates (sweep.py:488-532: dead rows keep their old values).    */
/* grad = grad_field[dst] * activation[src] (_sgd.py:118-119).                */
/* ------------------------------------------------------------------------ */

/* SGD: _sgd.py:121-126 -- w - lr * grad. */
OX_API void ox_update_sgd(int64_t cap, const int32_t* from, const int32_t* to,
                          const uint8_t* dead, float* w, const float* gfield,
                          const float* act, float lr) {
  #pragma omp parallel for schedule(static) if (cap >= OX_PAR_MIN)
  for (int64_t e = 0; e < cap; ++e) {
    if (dead[e]) continue;
    float grad = gfield[to[e]] * act[from[e]];
    w[e] = w[e] - lr * grad;
  }
}

/* Momentum: _momentum.py:136-139 -- v = mu*v + grad; w = w - lr*v. */
OX_API void ox_update_momentum(int64_t cap, const int32_t* from,
                               const int32_t* to, const uint8_t* dead, float* w,
                               float* vel, const float* gfield,
                               const float* act, float lr, float mu) {
  #pragma omp parallel for schedule(static) if (cap >= OX_PAR_MIN)
  for (int64_t e = 0; e < cap; ++e) {
    if (dead[e]) continue;
    float grad = gfield[to[e]] * act[from[e]];
    float v = mu * vel[e] + grad;
    vel[e] = v;
    w[e] = w[e] - lr * v;
  }
}

/* Adam(W): _adam.py:154-172, op for op. omb1/omb2 are float32(1 - b1),
 * float32(1 - b2) rounded from the double, as jnp.float32(1.0 - self.b1). */
OX_API void ox_update_adam(int64_t cap, const int32_t* from, const int32_t* to,
                           const uint8_t* dead, float* w, float* m, float* v,
                           float* t, const float* gfield, const float* act,
                           float lr, float b1, float b2, float eps, float wd,
                           float omb1, float omb2) {
  #pragma omp parallel for schedule(static) if (cap >= OX_PAR_MIN)
  for (int64_t e = 0; e < cap; ++e) {
    if (dead[e]) continue;
    float grad = gfield[to[e]] * act[from[e]];
    float weight = w[e];
    float step = t[e] + 1.0f;
    float mm = b1 * m[e] + omb1 * grad;
    float vv = b2 * v[e] + omb2 * (grad * grad);
    float m_hat = mm / (1.0f - ox_pow_step(b1, step));
    float v_hat = vv / (1.0f - ox_pow_step(b2, step));
    float dir = m_hat / (sqrtf(v_hat) + eps);
    float upd = lr * (dir + wd * weight);
    w[e] = weight - upd;
    m[e] = mm;
    v[e] = vv;
    t[e] = step;
  }
}

/* RMSProp: _rmsprop.py:135-140 -- ms = d*ms + (1-d)*g^2; w -= lr*g/sqrt(ms+eps). */
OX_API void ox_update_rmsprop(int64_t cap, const int32_t* from,
                              const int32_t* to, const uint8_t* dead, float* w,
                              float* ms, const float* gfield, const float* act,
                              float lr, float decay, float omd, float eps) {
  #pragma omp parallel for schedule(static) if (cap >= OX_PAR_MIN)
  for (int64_t e = 0; e < cap; ++e) {
    if (dead[e]) continue;
    float grad = gfield[to[e]] * act[from[e]];
    float s = decay * ms[e] + omd * (grad * grad);
    float upd = lr * grad / sqrtf(s + eps);
    w[e] = w[e] - upd;
    ms[e] = s;
  }
}

/* ------------------------------------------------------------------------ */
/* Free-slot accounting (phases.py:2573-2754): per-block dead counts and the  */
/* rank -> slot map "the r-th free slot in ascending slot order".            */
/* ------------------------------------------------------------------------ */

OX_API void ox_free_block_counts(int64_t cap, const uint8_t* dead,
                                 int32_t block, int32_t* counts) {
  int64_t nb = (cap + block - 1) / block;
  for (int64_t b = 0; b < nb; ++b) counts[b] = 0;
  for (int64_t e = 0; e < cap; ++e)
    if (dead[e]) counts[e / block] += 1;
}

/* slots[r] = the r-th dead slot (ascending) for r < n, or -1 past the end. */
OX_API int64_t ox_nth_free_slots(int64_t cap, const uint8_t* dead, int64_t n,
                                 int64_t* slots) {
  int64_t r = 0;
  for (int64_t e = 0; e < cap && r < n; ++e)
    if (dead[e]) slots[r++] = e;
  int64_t found = r;
  for (; r < n; ++r) slots[r] = -1;
  return found;
}

/* ------------------------------------------------------------------------ */
/* Site programs: the growth and pruning callbacks (propose, score,          */
/* importance, init, PruneConn predicate) that the reference evaluates under */
/* jax.vmap once per site (phases.py:3640-4058, :1444-1498). Registers hold  */
/* 32-bit patterns of float32 / int32 / uint32 / bool values; the opcodes    */
/* are listed in plastax_amd/_site.py (SOP). Integer semantics are jnp's     */
/* with 64-bit types off (wrapping int32/uint32, floor division and modulo,  */
/* saturating float->int casts with NaN -> 0). The rng draw of a site is     */
/* philox32(((keyed << 32) | key), (j << 16) | sub) (rng.py:206-259).         */
/* ------------------------------------------------------------------------ */

enum {
  S_CONST = 1, S_IDX = 2, S_LDU = 3, S_LDC = 4, S_RNG = 5, S_MOV = 6, S_SEL = 7,
  S_OUT = 8,
  S_FADD = 10, S_FSUB, S_FMUL, S_FDIV, S_FNEG, S_FABS, S_FMAX, S_FMIN, S_FTANH,
  S_FEXP, S_FLOG, S_FSQRT, S_FSIGMOID, S_FSQUARE, S_FRELU, S_FSIGN, S_FFLOOR,
  S_FCOS, S_FSIN,
  S_FGT = 30, S_FGE, S_FLT, S_FLE, S_FEQ, S_FNE,
  S_IADD = 40, S_ISUB, S_IMUL, S_INEG, S_IABS, S_IMAX, S_IMIN, S_IFLOORDIV,
  S_IMOD, S_ISIGN,
  S_IGT = 50, S_IGE, S_ILT, S_ILE, S_IEQ, S_INE,
  S_UMAX = 60, S_UMIN, S_UFLOORDIV, S_UMOD, S_UGT, S_UGE, S_ULT, S_ULE,
  S_AND = 70, S_OR, S_XOR, S_NOT, S_SHL, S_SHRU, S_SHRI, S_BNOT,
  S_I2F = 80, S_U2F, S_F2I, S_F2U, S_F2B, S_I2B,
  S_FLOG1P = 90, S_FEXPM1 = 91
};

#define OX_SREGS 32

static inline float ox_f(uint32_t b) { return ox_bits_to_float(b); }
static inline uint32_t ox_u(float f) { return ox_float_to_bits(f); }

static int32_t ox_floordiv_i32(int32_t a, int32_t b) {
  if (b == 0) return a == 0 ? -1 : -2; /* XLA's x/0 = -1, then jnp's floor fix */
  if (a == INT32_MIN && b == -1) return INT32_MIN;
  int32_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) q -= 1;
  return q;
}
static int32_t ox_mod_i32(int32_t a, int32_t b) {
  if (b == 0) return a;
  if (b == -1) return 0;
  int32_t r = a % b;
  if (r != 0 && ((r < 0) != (b < 0))) r += b;
  return r;
}
static int32_t ox_f2i(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return INT32_MAX;
  if (x <= -2147483648.0f) return INT32_MIN;
  return (int32_t)x;
}
static uint32_t ox_f2u(float x) {
  if (x != x || x <= 0.0f) return 0u;
  if (x >= 4294967296.0f) return UINT32_MAX;
  return (uint32_t)x;
}
static uint32_t ox_load32(const void* base, int32_t bytes, int64_t at) {
  if (bytes == 1) return ((const uint8_t*)base)[at] != 0;
  return ((const uint32_t*)base)[at];
}

/* Runs the program once for each of n sites. roles[r] (r = i, j, src, dst,
 * cid) is the role's per-site int32 array or NULL; key the per-site rng key
 * word or NULL; ufields/ubytes the unit columns (num_units long) and their
 * element sizes; cfields/cbytes the conn columns read at cid. Out slot k of
 * site s goes to outs[k][s]. */
OX_API void ox_site_eval(const int32_t* prog, int32_t ninstr, const uint32_t* consts,
                         int64_t n, const int32_t* const* roles, const uint32_t* key,
                         uint32_t keyed, const void* const* ufields,
                         const int32_t* ubytes, int64_t num_units,
                         const void* const* cfields, const int32_t* cbytes,
                         uint32_t* const* outs) {
  for (int64_t s = 0; s < n; ++s) {
    uint32_t r[OX_SREGS];
    memset(r, 0, sizeof r);
    int32_t ctx[5];
    for (int q = 0; q < 5; ++q) ctx[q] = roles[q] ? roles[q][s] : 0;
    uint64_t site_seed = ((uint64_t)keyed << 32) | (key ? key[s] : 0u);
    for (int32_t k = 0; k < ninstr; ++k) {
      const int32_t* q = prog + 4 * k;
      int32_t d = q[1], a = q[2], b = q[3];
      uint32_t x = r[a], y = r[b];
      int32_t xi = (int32_t)x, yi = (int32_t)y;
      switch (q[0]) {
        case S_CONST: r[d] = consts[a]; break;
        case S_IDX: r[d] = (uint32_t)ctx[a]; break;
        case S_LDU: {
          int64_t at = (int32_t)y;
          if (at < 0) at = 0;
          if (at > num_units - 1) at = num_units - 1;
          r[d] = ox_load32(ufields[a], ubytes[a], at);
          break;
        }
        case S_LDC: r[d] = ox_load32(cfields[a], cbytes[a], ctx[4]); break;
        case S_RNG:
          r[d] = ox_philox32(site_seed, ((uint64_t)(uint32_t)ctx[1] << 16) | (uint32_t)a);
          break;
        case S_MOV: r[d] = x; break;
        case S_SEL: r[d] = x ? r[b] : r[b + 1]; break;
        case S_OUT: outs[d][s] = x; break;
        case S_FADD: r[d] = ox_u(ox_f(x) + ox_f(y)); break;
        case S_FSUB: r[d] = ox_u(ox_f(x) - ox_f(y)); break;
        case S_FMUL: r[d] = ox_u(ox_f(x) * ox_f(y)); break;
        case S_FDIV: r[d] = ox_u(ox_f(x) / ox_f(y)); break;
        case S_FNEG: r[d] = x ^ 0x80000000u; break;
        case S_FABS: r[d] = x & 0x7FFFFFFFu; break;
        case S_FMAX: r[d] = ox_u(ox_fmax_nan(ox_f(x), ox_f(y))); break;
        case S_FMIN: r[d] = ox_u(ox_fmin_nan(ox_f(x), ox_f(y))); break;
        case S_FTANH: r[d] = ox_u(ox_tanhf(ox_f(x))); break;
        case S_FEXP: r[d] = ox_u(ox_expf(ox_f(x))); break;
        case S_FLOG: r[d] = ox_u(ox_logf(ox_f(x))); break;
        case S_FSQRT: r[d] = ox_u(sqrtf(ox_f(x))); break;
        case S_FSIGMOID: r[d] = ox_u(ox_sigmoidf(ox_f(x))); break;
        case S_FCOS: r[d] = ox_u(ox_cosf(ox_f(x))); break;
        case S_FSIN: r[d] = ox_u(ox_sinf(ox_f(x))); break;
        case S_FLOG1P: r[d] = ox_u(ox_log1pf(ox_f(x))); break;
        case S_FEXPM1: r[d] = ox_u(ox_expm1f(ox_f(x))); break;
        case S_FSQUARE: r[d] = ox_u(ox_f(x) * ox_f(x)); break;
        case S_FRELU: r[d] = ox_u(ox_fmax_nan(ox_f(x), 0.0f)); break;
        case S_FSIGN: {
          float v = ox_f(x);
          r[d] = v > 0.0f ? ox_u(1.0f) : (v < 0.0f ? ox_u(-1.0f) : x);
          break;
        }
        case S_FFLOOR: r[d] = ox_u(floorf(ox_f(x))); break;
        case S_FGT: r[d] = ox_f(x) > ox_f(y); break;
        case S_FGE: r[d] = ox_f(x) >= ox_f(y); break;
        case S_FLT: r[d] = ox_f(x) < ox_f(y); break;
        case S_FLE: r[d] = ox_f(x) <= ox_f(y); break;
        case S_FEQ: r[d] = ox_f(x) == ox_f(y); break;
        case S_FNE: r[d] = ox_f(x) != ox_f(y); break;
        case S_IADD: r[d] = x + y; break;
        case S_ISUB: r[d] = x - y; break;
        case S_IMUL: r[d] = x * y; break;
        case S_INEG: r[d] = 0u - x; break;
        case S_IABS: r[d] = xi < 0 ? 0u - x : x; break;
        case S_IMAX: r[d] = xi > yi ? x : y; break;
        case S_IMIN: r[d] = xi < yi ? x : y; break;
        case S_IFLOORDIV: r[d] = (uint32_t)ox_floordiv_i32(xi, yi); break;
        case S_IMOD: r[d] = (uint32_t)ox_mod_i32(xi, yi); break;
        case S_ISIGN: r[d] = (uint32_t)(xi > 0 ? 1 : (xi < 0 ? -1 : 0)); break;
        case S_IGT: r[d] = xi > yi; break;
        case S_IGE: r[d] = xi >= yi; break;
        case S_ILT: r[d] = xi < yi; break;
        case S_ILE: r[d] = xi <= yi; break;
        case S_IEQ: r[d] = x == y; break;
        case S_INE: r[d] = x != y; break;
        case S_UMAX: r[d] = x > y ? x : y; break;
        case S_UMIN: r[d] = x < y ? x : y; break;
        case S_UFLOORDIV: r[d] = y ? x / y : UINT32_MAX; break;
        case S_UMOD: r[d] = y ? x % y : x; break;
        case S_UGT: r[d] = x > y; break;
        case S_UGE: r[d] = x >= y; break;
        case S_ULT: r[d] = x < y; break;
        case S_ULE: r[d] = x <= y; break;
        case S_AND: r[d] = x & y; break;
        case S_OR: r[d] = x | y; break;
        case S_XOR: r[d] = x ^ y; break;
        case S_NOT: r[d] = ~x; break;
        case S_BNOT: r[d] = x == 0u; break;
        case S_SHL: r[d] = y >= 32u ? 0u : x << y; break;
        case S_SHRU: r[d] = y >= 32u ? 0u : x >> y; break;
        case S_SHRI:
          r[d] = y >= 32u ? (xi < 0 ? UINT32_MAX : 0u) : (uint32_t)(xi >> y);
          break;
        case S_I2F: r[d] = ox_u((float)xi); break;
        case S_U2F: r[d] = ox_u((float)x); break;
        case S_F2I: r[d] = (uint32_t)ox_f2i(ox_f(x)); break;
        case S_F2U: r[d] = ox_f2u(ox_f(x)); break;
        case S_F2B: r[d] = ox_f(x) != 0.0f; break;
        case S_I2B: r[d] = x != 0u; break;
        default: break;
      }
    }
  }
}
