/*
 * plastax_hip.h -- C ABI of the MI355X-native edge-arena step.
 *
 * The reference (Sir-NoChill/plastax) runs its streaming step as one jitted
 * JAX function whose edge work goes through XLA scatters or jax_triton custom
 * calls. This library is the drop-in for that edge work: each entry point
 * below replaces one reference seam (cited file:line), takes plain device
 * pointers and sizes, owns no memory, launches stream-ordered HIP kernels for
 * gfx950 and never synchronises the host. A return value of 0 means success;
 * any other value is a PLX_ERR_* code and plx_last_error() gives the text
 * (thread-local). No C++ exception crosses this boundary.
 *
 * Callers: plastax_amd/_lib.py (ctypes over torch-allocated device memory);
 * a jax.ffi / XLA custom-call handler would pass its buffers' device pointers
 * and its stream to the same entry points.
 */
#ifndef PLASTAX_HIP_H_
#define PLASTAX_HIP_H_

#ifndef __HIPCC_RTC__
#include <stdint.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define PLX_EXPORT __attribute__((visibility("default")))
#else
#define PLX_EXPORT
#endif

#define PLX_OK 0
#define PLX_ERR_INVALID 1     /* bad argument (shape, null pointer, range)   */
#define PLX_ERR_HIP 2         /* a HIP runtime call failed                   */
#define PLX_ERR_UNSUPPORTED 3 /* a policy or size this library cannot run    */

/* Named monoids (monoid.py:22-39). */
#define PLX_MONOID_SUM 0
#define PLX_MONOID_PROD 1
#define PLX_MONOID_MAX 2
#define PLX_MONOID_MIN 3

/* Per-edge update rules (optim/_sgd.py, _momentum.py, _adam.py, _rmsprop.py). */
#define PLX_RULE_SGD 0
#define PLX_RULE_MOMENTUM 1
#define PLX_RULE_ADAM 2
#define PLX_RULE_RMSPROP 3

#define PLX_MAX_INSTR 48
#define PLX_MAX_CONST 32
#define PLX_MAX_FIELDS 8
#define PLX_MAX_OUTS 4

/* A traced per-unit program: a user Apply (sweep.py:183-230) or the per-output
 * term of an elementwise Loss (phases.py:1107-1131). Opcodes are listed in
 * plastax_amd/_expr.py; each instruction is {op, dst, a, b}. LDU operand a
 * indexes `fields`; OUT slot d writes `outs[d]` at the unit. Passed by value
 * (it travels in the kernel argument segment).
 * fixed_mask (loss programs only; 0 elsewhere): bit k set means fields[k]
 * already points at one fixed unit's row (a loss reading u[F, UnitIdx(k)],
 * as the reference's examples/swifttd.py:381-392 does) and is read at the
 * sample index (0 in a streaming step), not at the output's unit. */
typedef struct plx_program {
  int32_t ninstr;
  int32_t nout;
  int32_t nfields;
  int32_t fixed_mask;
  int32_t code[4 * PLX_MAX_INSTR];
  float consts[PLX_MAX_CONST];
  const float* fields[PLX_MAX_FIELDS];
  float* outs[PLX_MAX_OUTS];
} plx_program;

/* Which units a pass finalizes (phases.py:1011, :1096-1101, sweep.py:205-207):
 * unit u finalizes iff (fin_level < 0 || level[u] == fin_level)
 * && !(skip_inputs && is_input[u]) && !(pruned && pruned[u]). level and
 * is_input are required; pruned may be null. */
typedef struct plx_finalize {
  const int32_t* level;
  const uint8_t* is_input;
  const uint8_t* pruned; /* null: the net has no unit capacity */
  int32_t fin_level;
  int32_t skip_inputs;
} plx_finalize;

/* A pass's map, of the product form (connection factor) * (unit factor at
 * the edge's other end): the reference's linear_input contract
 * c[WEIGHT, cid] * u[F, other] (phases.py:535-556) and its variants with a
 * constant factor (a constant map counts live edges: the in- or out-degree
 * under sum_). With PLX_MAP_W_CONST the connection factor of every edge is
 * `w` instead of WEIGHT; with PLX_MAP_X_CONST the unit factor is `x`
 * instead of the gathered field, whose pointer must still name a readable
 * unit column. flags 0 (a zeroed struct) is the linear map. */
#define PLX_MAP_W_CONST 1
#define PLX_MAP_X_CONST 2
typedef struct plx_map {
  int32_t flags;
  float w;
  float x;
  int32_t reserved;
} plx_map;

/* One bucket of the forward pass: _accumulate_into + _apply_masked
 * (sweep.py:113-230, phases.py:972-1015) for a linear map
 * weight * x[from] (phases.py:535-556). Rows are destination units in a CSR
 * over the physical (destination-sorted) positions; each row is folded in slot
 * order, combined into acc, and finalized rows apply `apply` and reset acc.
 * `dead` may be null when no row range holds a tombstone. */
struct plx_site_prog;

typedef struct plx_forward_desc {
  int32_t nrows;
  int32_t monoid;
  int32_t tbl_base; /* x[tbl_base, tbl_base + tbl_len) is staged in LDS    */
  int32_t tbl_len;  /* (at most 8192; 0: none)                             */
  const int32_t* row_unit; /* [nrows] destination unit ids, ascending      */
  const int32_t* row_ptr;  /* [nrows+1] physical positions                 */
  const int32_t* src;      /* [positions] FROM_ID                          */
  const float* weight;     /* [positions] WEIGHT                           */
  const uint8_t* dead;     /* [positions] DEAD                             */
  const float* x;          /* [num_units] the map's linear_input field     */
  float* acc;              /* [num_units] carried accumulator, or null     */
  plx_finalize fin;
  plx_program apply;
  plx_map map;             /* the map's factors (zeroed: weight * x[from]) */
  /* Optional (null prune_prog: none): a PruneConn predicate evaluated in the
   * same sweep (the fused forward + prune of phases.py:2322-2444). For every
   * position p of the rows' ranges, prune_sink[p] = 1 where the predicate
   * holds and p is not a tombstone (dead, when given), else 0; the predicate
   * is the site program at *prune_prog (device memory) evaluated as the
   * PLX_SITES_EDGE site s = p - prune_base with cid prune_slot[s] and unit
   * ids mapped through ids_logical / ids_physical (see plx_site_desc). The
   * state's DEAD is not written: the caller commits the sink at its prune
   * slot (plx_merge_kills). */
  const struct plx_site_prog* prune_prog;
  uint8_t* prune_sink;
  const int32_t* prune_slot;
  const int32_t* ids_logical;
  const int32_t* ids_physical;
  int64_t prune_base;
  int32_t num_units;
  int32_t reserved;
} plx_forward_desc;

PLX_EXPORT int plx_forward_bucket(const plx_forward_desc* d, void* stream);

/* Backward pass over one bucket, fused with the connection update
 * (phases.py:1049-1104 accumulating into FROM_ID; phases.py:1196-1242).
 * The bucket's physical positions [base, end) are split into nsuper
 * superblocks of consecutive tiles (super_tile[k] .. super_tile[k+1]); tile t
 * covers positions base + tile_pos[t] .. base + tile_pos[t+1] (at most
 * tile_size, multiples of 4). One workgroup walks each superblock in tile
 * order. With `fold`, every live edge's backward
 * term weight * g[dst] (pre-update weight) is folded per (tile, source)
 * group, in physical order, into a tile partial: a hot source (physical id
 * hot_base + h, h < nhot) has its tile partial folded, in tile order, into
 * its superblock sum, stored at hot_sb[superblock * nhot + h] (the identity
 * where the source is absent); the other sources' tile partials are stored
 * in their cold_partial slot. With
 * `update`, the same pass applies the update rule (see plx_update_desc for
 * p[] and the state columns) with grad = gfield[dst] * act[src] and stores
 * the new weight and state; dead edges keep theirs. Tile metadata:
 * sorted_rank[p - base] is, in its low 12 bits, the rank of position p
 * (below live_end) in its tile's (source, position) order, and bit 15 is set
 * where that rank starts a (tile, source) group; the hot sources' ranks are
 * [hlo, hhi) of the tile. grp_off[tile..tile+1] ranges the tile's groups in
 * grp, each packing its first rank (low 12 bits) and its length (high 4
 * bits; 15 means 15 or more: the group then ends at the next rank that
 * starts one, or at the tile's last ranked position). tile_info holds 16 int32 per tile: [0] hlo | hhi <<
 * 16; [1..7] the region bounds b1..b7; [8..15] the region offsets o0..o7.
 * A cold group starting at rank r stores its partial at o[x] + c, where c is
 * r, less hhi - hlo when r >= hhi, and x is the number of bounds b1..b7 at or
 * below c. tile_size is at most 4096; nhot at most 32767. */
typedef struct plx_tile_desc {
  int64_t base;
  int64_t end;
  int32_t tile_size;
  int32_t ntiles;
  int32_t nsuper;
  int32_t monoid;
  int32_t fold;
  int32_t update;
  int32_t nhot;
  int32_t rule;
  int32_t pow_table_len;
  int32_t tbl_base; /* act[tbl_base, tbl_base + tbl_len) is staged in LDS  */
  int32_t tbl_len;  /* (at most 8192; 0: none)                             */
  int32_t hot_base; /* hot sources are hot_base .. hot_base + nhot - 1     */
  int64_t live_end; /* with dead == null: positions >= live_end are dead   */
  int32_t step_mode; /* Adam: 0 per-edge step count s2; 1 every live edge  */
  float step_t;      /* has the step count step_t (s2 neither read nor      */
                     /* written; the caller advances step_t after the call) */
  const int32_t* tile_pos;   /* [ntiles+1] tile starts relative to base   */
  const int32_t* super_tile; /* [nsuper+1] first tile of each superblock  */
  const int32_t* tile_info;    /* [ntiles * 16] (fold)                     */
  const int32_t* grp_off;      /* [ntiles + 1] (fold)                      */
  const uint16_t* grp;         /* [groups] (fold)                          */
  const uint16_t* sorted_rank;
  float* hot_sb;
  float* cold_partial;
  const int32_t* src;
  const int32_t* dst;
  const uint8_t* dead;
  float* weight;
  float* s0;
  float* s1;
  float* s2;
  const float* g;       /* the backward map's linear_input field         */
  /* Optional (null: TO_ID is read from dst): with positions sorted by
   * destination, blk_dst0[(p - base) >> 12] + dst8[p - base] is TO_ID of
   * every position p below live_end (one byte per position instead of four;
   * blocks of 4,096 positions). */
  const uint8_t* dst8;
  const int32_t* blk_dst0;
  const float* gfield;  /* the update rule's grad field                  */
  const float* act;     /* ACTIVATION                                    */
  const float* pow_table;
  float p[8];
  plx_map map;          /* the backward map's factors (zeroed: weight * g[to]) */
} plx_tile_desc;

PLX_EXPORT int plx_backward_tiles(const plx_tile_desc* d, void* stream);

/* Backward finalize of one level from the partials of plx_backward_tiles.
 * A source's sum is the fold, in superblock order, of its superblock sums,
 * each the fold in tile order of its tile partials. Rows [0, nhot) are the hot
 * sources in hot-column order (row_hot[r] == r: column r of hot_sb, nsuper
 * rows of nhot); the others are cold (row_hot[r] == -1), finalized by
 * nparts workgroups, the k-th taking rows [part_rows[k], part_rows[k+1])
 * (at most 256; part_rows[0] == nhot when row_hot is given, else 0) (its run cold_partial[row_cold[r] .. row_cold[r+1])
 * in tile order, with each partial's superblock in cold_sb). The sum is
 * combined into acc (null: a fresh identity) and, where finalized, `apply`
 * runs and acc resets (sweep.py:183-230). Null row_hot / row_cold: rows fold
 * nothing (the deepest level, primed from the identity: phases.py:1089-1094). */
typedef struct plx_partials_desc {
  int32_t nrows;
  int32_t monoid;
  int32_t nsuper;
  int32_t nhot;
  int32_t nparts;
  int32_t reserved;
  const int32_t* part_rows;
  const int32_t* row_unit;
  const int32_t* row_hot;
  const int32_t* row_cold;
  const float* hot_sb;
  const float* cold_partial;
  const uint16_t* cold_sb;
  const int32_t* cold_idx;
  float* acc;
  plx_finalize fin;
  plx_program apply;
  /* optional [nparts][4]: each cold workgroup's first row, end row and first
   * and end cold entry (row_cold at those rows), read in one load */
  const int32_t* part_info;
} plx_partials_desc;

PLX_EXPORT int plx_backward_partials(const plx_partials_desc* d, void* stream);

/* Source-value tables: a bucket's sources are renumbered most-used first,
 * so the values of its busiest sources are one contiguous slice of the
 * gathered column; kernels copy that slice into LDS once per workgroup and
 * gather those sources from it (bit-identical values, fewer cache requests). */
#define PLX_MAX_TBL 8192

/* Connection update over physical positions [0, n): build_update_conn_phase
 * (phases.py:1196-1242, sweep.py:488-532) for the optim bundles. grad =
 * gfield[dst] * act[src]; dead rows keep their values.
 *   SGD:      p0=lr                          (_sgd.py:121-126)
 *   MOMENTUM: p0=lr p1=mu           s0=opt/v (_momentum.py:136-139)
 *   ADAM:     p0=lr p1=b1 p2=b2 p3=eps p4=wd p5=1-b1 p6=1-b2;
 *             s0=opt/m s1=opt/v s2=opt/t     (_adam.py:154-172)
 *   RMSPROP:  p0=lr p1=decay p2=1-decay p3=eps  s0=opt/v (_rmsprop.py:135-140)
 * pow_table (optional, Adam) holds float32(b1^t), float32(b2^t) at [2t], [2t+1]
 * for t < pow_table_len; other t are computed on the device the same way.
 * `dead` may be null: positions >= live_end are then the dead ones. */
typedef struct plx_update_desc {
  int64_t n;
  int32_t rule;
  int32_t pow_table_len;
  int32_t tbl_base; /* act[tbl_base, tbl_base + tbl_len) is staged in LDS  */
  int32_t tbl_len;  /* (at most 8192; 0: none)                             */
  int64_t live_end; /* with dead == null: positions >= live_end are dead   */
  int32_t step_mode; /* as plx_tile_desc                                   */
  float step_t;
  const int32_t* src;
  const int32_t* dst;
  const uint8_t* dead;
  float* weight;
  float* s0;
  float* s1;
  float* s2;
  const float* gfield;
  const float* act;
  const float* pow_table;
  /* Optional, as plx_tile_desc's (positions here start at 0):
   * blk_dst0[p >> 12] + dst8[p] is TO_ID below live_end. */
  const uint8_t* dst8;
  const int32_t* blk_dst0;
  float p[8];
} plx_update_desc;

PLX_EXPORT int plx_update_conn(const plx_update_desc* d, void* stream);

/* ---- Batched steps (make_step(batch_size=B): step.py:359-468) ----------
 * Unit columns of a batched step are [num_units][B] (sample b of unit u at
 * u * B + b); every per-sample fold keeps the streaming step's order.
 *
 * Forward of one bucket for B samples (phases.py:812-840 with the per-sample
 * edge list's order): plx_forward_bucket's descriptor with x, acc and the
 * apply program's fields and outs batched; tbl_* are ignored. Row r folds
 * its positions in slot order per sample. */
PLX_EXPORT int plx_forward_batch(const plx_forward_desc* d, int32_t batch, void* stream);

/* Backward of one bucket for B samples (build_csr_backward, phases.py:843-934,
 * and the reference's per-sample scatter order): row r is source unit
 * row_unit[r]; its out-edges are the list entries j in [row_ptr[r],
 * row_ptr[r+1]) in logical slot order, entry j contributing weight[j] *
 * g[dst[j] * B + b] (pre-update weights) where live[j] is nonzero, folded in
 * that order from the identity, combined into acc (null: the identity) and,
 * where the row finalizes, `apply` runs (fields and outs batched) and acc
 * resets. The lists are slot-ordered copies of the arena's columns
 * (plx_gather_edges); a factor the map holds constant (plx_map flags) is
 * not loaded, so its copy need not exist. */
typedef struct plx_bwd_batch_desc {
  int32_t nrows;
  int32_t monoid;
  int32_t batch;
  int32_t reserved;
  const int32_t* row_unit;
  const int32_t* row_ptr;
  const int32_t* dst;    /* [entries] TO_ID */
  const float* weight;   /* [entries] WEIGHT */
  const uint8_t* live;   /* [entries] 0: skipped (null: every entry live) */
  const float* g;        /* [num_units][B] the map's linear_input field */
  float* acc;            /* [num_units][B] carried accumulator, or null */
  plx_finalize fin;
  plx_program apply;
  plx_map map;           /* the map's factors (zeroed: weight * g[dst]) */
} plx_bwd_batch_desc;

PLX_EXPORT int plx_backward_batch(const plx_bwd_batch_desc* d, void* stream);

/* The streaming backward of one bucket over the same slot-ordered lists
 * (batch must be 1): one lane per row, each folding its list in slot order
 * (the reference's per-source scatter order, sweep.py:343-399). Used by the
 * churn layout, which rebuilds on the device after every structural change. */
PLX_EXPORT int plx_backward_lists(const plx_bwd_batch_desc* d, void* stream);

/* out_weight[j] = weight[pos[j]] (out_weight optional), out_live[j] =
 * !dead[pos[j]] (out_live optional; dead null: all live) for j < n: a
 * bucket's backward lists in slot order. */
PLX_EXPORT int plx_gather_edges(int64_t n, const int32_t* pos, const float* weight, const uint8_t* dead,
                                float* out_weight, uint8_t* out_live, void* stream);

/* The exact batched connection update (build_batched_update_conn,
 * phases.py:390-483): per live position, stat_b = gfield[dst * B + b] *
 * act[src * B + b]; total = stat_0, then total + stat_b for b = 1 .. B-1;
 * mean = total / B; then the update rule of plx_update_conn with grad =
 * mean (tbl_* ignored; gfield and act batched). */
PLX_EXPORT int plx_update_batch(const plx_update_desc* d, int32_t batch, void* stream);

/* The same update with the edges grouped into tiles of at most 64
 * destination x 64 source units (tile k: entries tile_off[k] ..
 * tile_off[k+1], at most 1,024; destination ids tile_base[2k] + 0..63,
 * source ids tile_base[2k+1] + 0..63), so a workgroup stages its tile's
 * unit rows through LDS, 64 samples at a time, and each edge reads them from
 * there. Entry j is the edge at position pos[j] (relative to d's columns),
 * loc[j] = (dst - dst base) | (src - src base) << 8. Every live edge of
 * [0, d->n) appears once; the sum over the samples keeps the order of
 * plx_update_batch (stat_0 + stat_1 + ...), so the results are the same
 * bits. num_units bounds the staged rows. No counterpart in the reference:
 * a layout of plx_update_batch's work. */
typedef struct plx_batch_tiles {
  int32_t ntiles;
  int32_t num_units;
  const int32_t* tile_off;  /* [ntiles + 1] */
  const int32_t* tile_base; /* [2 * ntiles] */
  const int32_t* pos;       /* [entries] */
  const uint16_t* loc;      /* [entries] */
} plx_batch_tiles;

/* The tile limits plx_update_batch_tiles is built with: units per tile side
 * (loc's fields index [0, *rows)) and edges per tile (entries beyond are not
 * updated). Table builders check theirs against these. */
PLX_EXPORT int plx_batch_tile_limits(int32_t* rows, int32_t* edges);

/* Roof probes (no counterpart in the reference: a measurement helper for
 * the benchmark's rooflines). Times one launch of a read loop and returns
 * the bytes it read and its duration (the call synchronises `stream`):
 * PLX_PROBE_LDS, conflict-free 16-byte LDS reads (buf unused); PLX_PROBE_L2,
 * coalesced 16-byte reads of buf (buf_bytes / 16 a power of two; a few MB
 * stay L2-resident). out: 2048 * 256 uint32 of device memory. */
#define PLX_PROBE_LDS 0
#define PLX_PROBE_L2 1
PLX_EXPORT int plx_roof_probe(int32_t kind, int32_t iters, const void* buf, int64_t buf_bytes, uint32_t* out,
                              double* bytes, float* ms, void* stream);

PLX_EXPORT int plx_update_batch_tiles(const plx_update_desc* d, const plx_batch_tiles* t, int32_t batch,
                                      void* stream);

/* Batched losses: sample b's outputs at ids[k] * B + b, targets[b * n_out +
 * k], loss into losses[b]; the per-sample fold is plx_loss_elementwise's /
 * plx_loss_softmax_ce's. partials: B * ceil(n_out / 256) floats. */
PLX_EXPORT int plx_loss_elementwise_batch(int32_t n_out, const int32_t* output_ids,
                                          const float* targets, const plx_program* term,
                                          float* seed_field, float* partials, float* losses,
                                          int32_t batch, void* stream);
PLX_EXPORT int plx_loss_softmax_ce_batch(int32_t n_out, const int32_t* output_ids,
                                         const float* act, const float* targets,
                                         float* seed_field, float* losses, int32_t batch,
                                         void* stream);

/* StepResult.loss of a batched step (step.py:466): (0 + l_0 + ... + l_{B-1}) / B. */
PLX_EXPORT int plx_batch_mean(int32_t batch, const float* losses, float* out, void* stream);

/* reduce_batch_units (phases.py:298-332) for one column: dst[u] from
 * src[u * B .. u * B + B): PLX_REDUCE_MEAN (float32: x_0 + x_1 + ... in
 * sample order, then / B), PLX_REDUCE_SUM (the same sum; int32 wraps),
 * PLX_REDUCE_FIRST (x_0). kind: PLX_COL_F32, PLX_COL_I32 (MEAN refused) or
 * PLX_COL_U8 (FIRST only). */
#define PLX_REDUCE_MEAN 0
#define PLX_REDUCE_SUM 1
#define PLX_REDUCE_FIRST 2
#define PLX_COL_F32 0
#define PLX_COL_I32 1
#define PLX_COL_U8 2
PLX_EXPORT int plx_reduce_batch(int64_t n, int32_t batch, int32_t mode, int32_t kind,
                                const void* src, void* dst, void* stream);

/* Step input scatter (step.py:598): dst[ids[k]] = values[k]. */
PLX_EXPORT int plx_scatter_f32(int32_t n, const int32_t* ids, const float* values,
                    float* dst, void* stream);

/* Elementwise loss (phases.py:1107-1131 with a policy whose seed and loss
 * term are elementwise in (prediction, target), e.g. MSE): `term` writes out
 * slot 0 (the seed) to seed_field[output_ids[k]]; slot 1 is the loss term.
 * *loss_out = the fold of the terms in 256-output pieces (each piece folded
 * in order, then the piece sums in order). partials: ceil(n_out/256) floats
 * of scratch. */
PLX_EXPORT int plx_loss_elementwise(int32_t n_out, const int32_t* output_ids,
                         const float* targets, const plx_program* term,
                         float* seed_field, float* partials, float* loss_out,
                         void* stream);

/* SoftmaxCrossEntropyLoss (traits.py:204-250): max, sum of exp(a - max) in
 * 256-output pieces, seed = exp(z)/s - t, loss = piecewise fold of
 * t*(log s - z). Runs in one workgroup. */
PLX_EXPORT int plx_loss_softmax_ce(int32_t n_out, const int32_t* output_ids,
                        const float* act, const float* targets,
                        float* seed_field, float* loss_out, void* stream);

/* Fill n floats with a value (identity accumulators). */
PLX_EXPORT int plx_fill_f32(int64_t n, float value, float* dst, void* stream);

/* Device-side Philox-4x32-10 in the plastax mapping (rng.py:109-141):
 * out[i] = philox32(seeds[i], ctrs[i]). Used to pin the device generator. */
PLX_EXPORT int plx_philox32(int64_t n, const uint64_t* seeds, const uint64_t* ctrs,
                 uint32_t* out, void* stream);

/* Elementary functions exactly as the kernels evaluate them (op 0 exp,
 * 1 log, 2 tanh, 3 sigmoid, 4 sqrt, 5 Adam power b^t with b=x[i], t=y[i],
 * 6 cos, 7 sin, 8 log1p, 9 expm1). */
PLX_EXPORT int plx_eval_math(int32_t op, int64_t n, const float* x, const float* y,
                  float* out, void* stream);

/* sizeof of the descriptor structs, in the order plx_program, plx_finalize,
 * plx_forward_desc, plx_tile_desc, plx_partials_desc, plx_update_desc,
 * plx_site_prog, plx_site_desc, plx_sort_key, plx_sort_desc,
 * plx_grow_filter_desc, plx_grow_col, plx_grow_claim_desc, plx_unit_col,
 * plx_bwd_batch_desc, plx_batch_tiles, plx_tile_build_desc, plx_gen_fold_desc,
 * plx_merge_desc, plx_merge_gather_desc (for binding layers to check their
 * mirrors). Writes min(n, 20) values and returns 20. */
PLX_EXPORT int plx_struct_sizes(int64_t* out, int32_t n);

/* ========================================================================
 * Structural phases: PruneConn and add_conn growth (plastax_amd/csrc/
 * structural.hip). They work on the *logical* arena: every bucket's columns
 * in slot order, concatenated bucket after bucket into flat columns (bucket
 * b at [off_b, off_b + cap_b)), unit ids in the caller's numbering.
 * ======================================================================== */

#define PLX_MAX_SINSTR 160
#define PLX_MAX_SCONST 32
#define PLX_MAX_SFIELDS 8
#define PLX_MAX_SOUTS 8

/* A traced growth / pruning callback (propose, score, importance, init,
 * PruneConn predicate: phases.py:3640-4058, :1444-1498). 32-bit registers
 * hold float32 / int32 / uint32 / bool values; opcodes are listed in
 * plastax_amd/_site.py (SOP). Unit field f is read at an int index clamped
 * to [0, num_units); conn field f at the site's cid. ubytes/cbytes: 4, or 1
 * for byte (bool) columns. */
typedef struct plx_site_prog {
  int32_t ninstr;
  int32_t nout;
  int32_t reserved[2];
  int32_t code[4 * PLX_MAX_SINSTR];
  uint32_t consts[PLX_MAX_SCONST];
  const void* ufields[PLX_MAX_SFIELDS];
  const void* cfields[PLX_MAX_SFIELDS];
  int32_t ubytes[PLX_MAX_SFIELDS];
  int32_t cbytes[PLX_MAX_SFIELDS];
} plx_site_prog;

/* How site s maps to the roles (i, j, src, dst, cid) and the rng key. */
#define PLX_SITES_UNIT 0   /* i = s / per, j = s % per; key i (per-unit proposals, importance) */
#define PLX_SITES_GLOBAL 1 /* j = s; key 0 (phases.py:3766-3810) */
#define PLX_SITES_CONN 2   /* r = s / per, j = s % per, cid = list_a[r];
                              key conn_key(from_id[cid], to_id[cid], occ[cid]) */
#define PLX_SITES_GRID 3   /* g = s / per^2: src = list_a[g per + a], dst = list_b[g per + b],
                              with s % per^2 = a per + b (candidate grids) */
#define PLX_SITES_PAIRS 4  /* src = list_a[s], dst = list_b[s] (init of the winners) */
#define PLX_SITES_EDGE 5   /* cid = s; src = from_id[s], dst = to_id[s] when given (through
                              ids_logical when set): PruneConn, UpdateConn */

/* One evaluation of a site program over n sites (replaces the jax.vmap of a
 * growth / pruning callback). The rng of a site is philox32(((keyed << 32)
 * | key), (j << 16) | sub) with keyed = philox32(net_seed, (step << 8) | 1)
 * (rng.py:206-259). Out slot k of site s is written to outs[k][s] (32-bit
 * patterns); with or_into set, slot 0 is instead OR-ed into that byte column
 * (dead |= predicate) and kill_count (optional) counts the bytes it turned
 * from 0 to 1. n_dev, when set, holds the site count (<= n).
 *
 * Renumbered storage: the program always sees the caller's unit ids and
 * logical slots. With ids_physical set, a unit field read at id u reads
 * position ids_physical[u]; a conn field whose cbytes has PLX_SITE_ID_COLUMN
 * holds physical unit ids and reads back ids_logical[value]; with site_ids
 * set, the cid (EDGE sites) or unit i (UNIT sites) the program sees is
 * site_ids[s] (site_ids[s / per]) while fields are read at the site's own
 * position. */
#define PLX_SITE_ID_COLUMN 0x100
typedef struct plx_site_desc {
  plx_site_prog prog;
  int64_t n;
  int32_t kind;
  int32_t per;
  int32_t num_units;
  int32_t step;
  uint64_t net_seed;
  const int32_t* list_a;
  const int32_t* list_b;
  const int32_t* from_id;
  const int32_t* to_id;
  const int32_t* occ;
  const int32_t* n_dev;
  void* outs[PLX_MAX_SOUTS];
  uint8_t* or_into;
  int32_t* kill_count;
  const int32_t* site_ids;
  const int32_t* ids_logical;
  const int32_t* ids_physical;
  /* batch > 1: the unit columns are [num_units][batch] (a batched step's
   * per-sample columns) and a unit read at unit u reads u * batch + b, b the
   * site's sample: for PLX_SITES_UNIT the n = num_units * batch sites are
   * (unit s / batch, sample s % batch) and out slot k of site s lands at
   * outs[k][s] (with site_ids: n is a multiple of batch and the unit is
   * site_ids[s / batch]); for the other kinds b is `sample`. */
  int32_t batch;
  int32_t sample;
  /* With or_into: stamp (optional) gets stamp_value at every site whose
   * byte turns to 1 (see plx_kill_incident). */
  float* stamp;
  float stamp_value;
} plx_site_desc;

PLX_EXPORT int plx_site_eval(const plx_site_desc* d, void* stream);

/* A site program compiled to its own kernel: the same evaluation as
 * plx_site_eval (its instructions are the interpreter's, with literal
 * operands, so the results are the same bits), without interpreting the
 * program per site. The reference lowers the PruneConn predicate's jaxpr to
 * the fused kernel's source the same way (phases.py:1910-2147, template
 * :2174-2203). plx_site_compile generates the kernel's source for the
 * program of `d` and its launch shape (site kind, batched or not, which of
 * from_id / to_id / site_ids / ids_logical / ids_physical are set, the
 * fields' widths: fixed in the kernel, so its loads need no branch) and
 * compiles it with hipRTC for `arch` (null: the current device's), with the
 * library's floating-point flags, headers from `csrc_dir` (the library's csrc
 * directory); the module is loaded and *handle set, one compile per (device,
 * program code, shape) for the process. With handle null it only compiles (a
 * check that needs no device). plx_site_eval_compiled runs a handle on a
 * descriptor with the same code and shape (checked; the constants, counts and
 * pointers are the descriptor's). */
PLX_EXPORT int plx_site_compile(const plx_site_desc* d, const char* csrc_dir, const char* arch, void** handle);
PLX_EXPORT int plx_site_eval_compiled(void* handle, const plx_site_desc* d, void* stream);

/* The fused forward + PruneConn sweep with the predicate compiled in: the
 * reference translates the predicate's jaxpr into the fused forward kernel's
 * source (phases.py:1910-2147, template :2174-2203, launch :2240-2319).
 * plx_forward_prune_compile generates plx_forward_bucket's kernel for monoid
 * `monoid` (PLX_MONOID_*) with the program of `d` (an unbatched
 * PLX_SITES_EDGE program; d's ids_logical / ids_physical set as the forward
 * descriptor's will be, and its fields' widths) in place of the site
 * interpreter, compiled and cached as plx_site_compile does.
 * plx_forward_bucket_compiled runs a bucket on it: the same descriptor,
 * checks and results as plx_forward_bucket with that prune_prog, which must
 * hold the compiled program (its fields and constants are read from it; its
 * instructions are the compiled ones). */
PLX_EXPORT int plx_forward_prune_compile(const plx_site_desc* d, int32_t monoid, const char* csrc_dir,
                                         const char* arch, void** handle);
PLX_EXPORT int plx_forward_bucket_compiled(void* handle, const plx_forward_desc* d, void* stream);

/* One bucket of a generic pass (a map outside the product form, one float32
 * component or a tuple with a tuple of monoids: sweep.py:113-180 / :343-399
 * with any `map` and `combine`): for every row r (one thread each), unit u =
 * row_unit[r], its entries j in [row_ptr[r], row_ptr[r+1]) in order, each at
 * physical position p = entry_pos ? entry_pos[j] : j, skipped where dead[p]
 * (dead optional): the map program (`prog`, ncomp float32 outputs) runs as
 * the PLX_SITES_EDGE site s = p - base (its connection columns start at
 * base) with cid slot[s] and the unit ids seen through ids_logical (unit
 * reads through ids_physical); a forward row binds dst = u and src =
 * from_id[p], a backward row (backward != 0) src = u and dst = to_id[p].
 * Component k folds in entry order from identity[k] with monoid[k]
 * (PLX_MONOID_*), then acc[k][u] = monoid[k](acc[k][u], fold). */
typedef struct plx_gen_fold_desc {
  plx_site_prog prog;
  int32_t nrows;
  int32_t ncomp;
  int32_t backward;
  int32_t num_units;
  int32_t monoid[8];
  float identity[8];
  const int32_t* row_unit;
  const int32_t* row_ptr;
  const int32_t* entry_pos;
  const int32_t* from_id;
  const int32_t* to_id;
  const uint8_t* dead;
  int64_t base;
  const int32_t* slot;
  const int32_t* ids_logical;
  const int32_t* ids_physical;
  float* acc[8];
  /* samples (>= 1): unit columns and acc are [num_units][batch]; each
   * (row, sample) folds its entries with the unit reads at that sample */
  int32_t batch;
  int32_t reserved;
} plx_gen_fold_desc;

PLX_EXPORT int plx_gen_fold(const plx_gen_fold_desc* d, void* stream);

/* The mean-of-writes connection update of a batched step with a user
 * UpdateConn (phases.py:484-533), one float32 column at a time over n
 * slots: mode 0 total = next - old; mode 1 total = total + (next - old)
 * (samples in order); mode 2 old = old + total / batch. */
#define PLX_MOW_FIRST 0
#define PLX_MOW_ADD 1
#define PLX_MOW_APPLY 2
PLX_EXPORT int plx_mean_of_writes(int64_t n, int32_t mode, int32_t batch, float* old, const float* next,
                                  float* total, void* stream);

/* Ordered stream compaction (the free-slot accounting of phases.py:2573-2754
 * and every "which candidates survive" list): out[k] = the k-th position p
 * in [0, n) whose flag is set, ascending; *count = their number. Flag of p:
 * mode 0 u8[p] != 0, 1 u8[p] == 0, 2 f32[p] finite, 3 i32[p] != 0. n_dev
 * optional. scratch: plx_scratch_ints(n) ints. */
#define PLX_FLAG_U8 0
#define PLX_FLAG_U8_ZERO 1
#define PLX_FLAG_FINITE 2
#define PLX_FLAG_I32 3
PLX_EXPORT int plx_compact(int64_t n, const int32_t* n_dev, int32_t mode, const void* flags,
                           int32_t* out, int32_t* count, int32_t* scratch, void* stream);

/* Exclusive prefix sum of n int32 (n_dev optional); *total (optional) gets
 * the sum. scratch: plx_scratch_ints(n) ints. */
PLX_EXPORT int plx_scan_i32(int64_t n, const int32_t* n_dev, const int32_t* in, int32_t* out,
                            int32_t* total, int32_t* scratch, void* stream);

/* Scratch ints plx_compact / plx_scan_i32 / plx_sort need for n elements. */
PLX_EXPORT int64_t plx_scratch_ints(int64_t n);

/* plx_compact without a workspace: its chunk sums live in a file-scope
 * device array of PLX_COMPACT_NOALLOC_MAX_N / 2048 ints (128 KiB per GPU,
 * held until the process ends), so the call allocates nothing. No
 * counterpart in the reference: it is for callers that cannot allocate
 * (code under stream capture, serving loops, harnesses that forbid
 * hipMalloc). n > PLX_COMPACT_NOALLOC_MAX_N returns PLX_ERR_UNSUPPORTED.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (concurrent streams or threads) race. */
#define PLX_COMPACT_NOALLOC_MAX_N (1LL << 26)
PLX_EXPORT int plx_compact_noalloc(int64_t n, const int32_t* n_dev, int32_t mode, const void* flags,
                                   int32_t* out, int32_t* count, void* stream);

/* Sort keys, least significant first; each is derived from the index being
 * sorted (idx) and ordered ascending over its low `bits` bits:
 *   I32      a[idx] (int32 read as unsigned; callers keep it >= 0)
 *   SCORE    the total order's leading key of the float a[idx]: -score, NaN
 *            as +inf, -0 as +0 (phases.py:4200-4281), as an ordered uint32
 *   LEVEL_OF b[a[idx]] (a unit's level through an id column)
 *   PAIR16   (a[idx] << 16) | b[idx] (ids below 2^16)
 *   DEADMAX  dead-masked id: b (u8) [idx] ? bits-max : a[idx]  */
#define PLX_KEY_I32 0
#define PLX_KEY_SCORE 1
#define PLX_KEY_LEVEL_OF 2
#define PLX_KEY_PAIR16 3
#define PLX_KEY_DEADMAX 4
typedef struct plx_sort_key {
  int32_t kind;
  int32_t bits;
  int32_t bound; /* LEVEL_OF: ids clamped to [0, bound) when > 0 */
  int32_t reserved;
  const void* a;
  const void* b;
} plx_sort_key;

/* Stable LSD radix sort of an index list by up to 6 keys (8-bit digits,
 * 4096-element LDS-ranked tiles): the total order of phases.py:4237-4321
 * and the other sorts of the growth pipeline. vals (n_max, count in n_dev
 * or n_max) is sorted in place; keys/keys_alt/vals_alt are n_max uint32 of
 * scratch, hist plx_scratch_ints(n_max) ints. */
typedef struct plx_sort_desc {
  int64_t n_max;
  const int32_t* n_dev;
  int32_t nkeys;
  int32_t reserved;
  plx_sort_key keys[6];
  uint32_t* vals;
  uint32_t* keys_buf;
  uint32_t* keys_alt;
  uint32_t* vals_alt;
  int32_t* hist;
} plx_sort_desc;

PLX_EXPORT int plx_sort(const plx_sort_desc* d, void* stream);

/* Candidate validity (phases.py:4061-4153, :4776-4800): score[s] becomes
 * -inf unless the candidate (src[s], dst[s]) is in range (check_range:
 * proposals; out-of-range ids are clamped to 0, phases.py:4041-4058), its
 * proposer is live (proposer_dead[proposer_idx ? proposer_idx[s/per] :
 * s/per] == 0, when proposer_dead is set), both endpoints are live (pruned
 * optional), |level[dst] - level[src]| <= max_level_gap, the direction holds
 * (0 any, 1 deeper, 2 same_or_deeper), it is no self-loop unless allowed,
 * TOPOLOGICAL: level[src] is a bucket (and equals s / grid_sq when grid_sq >
 * 0, the per-level grids), and with nlive > 0 the pair is not a live edge of
 * its bucket: live_idx (count in nlive_dev, or nlive) lists the live flat
 * slots sorted by (bucket, src, dst) over live_bucket/live_src/live_dst. */
typedef struct plx_grow_filter_desc {
  int64_t n;
  int64_t grid_sq;
  int32_t num_units;
  int32_t num_buckets;
  int32_t pipeline;
  int32_t max_level_gap;
  int32_t direction;
  int32_t allow_self_loops;
  int32_t check_range;
  int32_t per;
  int32_t* src;
  int32_t* dst;
  float* score;
  const int32_t* level;
  const uint8_t* pruned;
  const int32_t* proposer_idx;
  const uint8_t* proposer_dead;
  int64_t nlive;            /* capacity of live_idx */
  const int32_t* nlive_dev; /* optional: the live count in device memory */
  const int32_t* live_idx;
  const int32_t* live_bucket;
  const int32_t* live_src;
  const int32_t* live_dst;
} plx_grow_filter_desc;

PLX_EXPORT int plx_grow_filter(const plx_grow_filter_desc* d, void* stream);

/* dedupe_step (phases.py:4156-4183): order lists candidate indices sorted by
 * (src, dst), stably over the score-descending order; every copy of a pair
 * after its first gets score -inf. */
PLX_EXPORT int plx_grow_mark_repeats(int64_t n_max, const int32_t* n_dev, const int32_t* order,
                                     const int32_t* src, const int32_t* dst, float* score,
                                     void* stream);

/* Selection (phases.py:4324-4469): sorted (n_max, count n_dev) lists
 * candidate indices in the total order, level-major when per_segment. A
 * candidate's segment is level[src[idx]]; with per_segment, the first k of
 * every segment win (first: num_segments ints of scratch), else the first k
 * overall. win[p] = 1 for winning positions. */
PLX_EXPORT int plx_grow_select(int64_t n_max, const int32_t* n_dev, const int32_t* sorted,
                               const int32_t* src, const int32_t* level, int32_t per_segment,
                               int64_t k, int32_t num_segments, int32_t* first, uint8_t* win,
                               void* stream);

/* The claim and write of the winners (phases.py:2853-3106, :4944-5110).
 * winners (n_max, count n_dev) lists candidate indices levels ascending, the
 * total order within a level. A winner is growable if its score is finite and
 * at least `threshold` (has_threshold); max_new_per_step (>0) caps the
 * growable ones in list order. Its rank among its own level's growable
 * winners picks its slot:
 *   TOPOLOGICAL (pipeline = 0): its source level's bucket's rank-th free
 *     slot: free_slots lists every dead flat slot ascending and bucket b's
 *     run of it is free_info[2b] (start), free_info[2b + 1] (length), as
 *     plx_bucket_free computes them;
 *   PIPELINE: the rank-th of its level's own dead slots (own_slots grouped
 *     by level, own_start / own_count per level), the rest spill to the tail
 *     at tail_start, levels ascending, up to capacity.
 * Committed winners write from_id, to_id, dead = 0 and every column in
 * cols: from init output slot (init_out[q] for winner q) or the column's
 * default bits. flags[0] += committed, flags[1] |= overflow, flags[2] |=
 * committed with level[dst] <= level[src], flags[3] += tail slots used
 * (flags[4]: see tail_dev). scratch: 8 n_max + plx_scratch_ints(n_max) ints. */
#define PLX_MAX_GROW_COLS 16
typedef struct plx_grow_col {
  void* ptr;
  int32_t bytes;
  int32_t init_slot; /* -1: write default_bits */
  uint32_t default_bits;
  int32_t reserved;
} plx_grow_col;

typedef struct plx_grow_claim_desc {
  int64_t n_max;
  const int32_t* n_dev;
  const int32_t* winners;
  const int32_t* src;
  const int32_t* dst;
  const float* score;
  const int32_t* level;
  int32_t pipeline;
  int32_t num_buckets;
  int32_t num_levels;
  int32_t has_threshold;
  float threshold;
  int32_t max_new_per_step;
  int64_t capacity;
  int64_t tail_start;
  const int32_t* free_slots;
  const int32_t* free_info;
  const int32_t* own_slots;
  const int32_t* own_start;
  const int32_t* own_count;
  int32_t* from_id;
  int32_t* to_id;
  uint8_t* dead;
  int32_t ncols;
  int32_t reserved;
  plx_grow_col cols[PLX_MAX_GROW_COLS];
  const uint32_t* init_out[PLX_MAX_SOUTS];
  int32_t* flags;
  int32_t* scratch;
  /* The same-step retry of an overflowing growth (phases.py:5206-5281):
   * with growable_in set, winner q is growable iff growable_in[q] != 0 (no
   * threshold or step cap: they were applied by the attempt). dropped_out
   * (optional) gets 1 for every growable winner that found no slot. */
  const int32_t* growable_in;
  int32_t* dropped_out;
  /* PIPELINE, optional: the tail start read from the device (int32)
   * instead of tail_start; flags then holds five ints and flags[4] gets the
   * new tail start, *tail_dev + flags[3], so a caller can pass &flags[4] as
   * the next claim's tail_dev without reading anything on the host. */
  const int32_t* tail_dev;
  /* Optional (null: none): every slot the claim fills is appended to
   * claimed_out (in no particular order) at index atomicAdd(claimed_n, 1);
   * the caller zeroes *claimed_n first. Appends at or past claimed_cap are
   * not written, so the caller sizes it by a bound on the claims (the
   * winners' budget). plx_claimed_split turns the list into each bucket's
   * claimed slots in ascending order. */
  int32_t* claimed_out;
  int32_t* claimed_n;
  int64_t claimed_cap;
} plx_grow_claim_desc;

PLX_EXPORT int plx_grow_claim(const plx_grow_claim_desc* d, void* stream);

/* The claimed slots of plx_grow_claim's list, split by bucket and sorted:
 * for bucket b (flat slots [offs[b], offs[b+1]); offs: nb + 1 int64 on the
 * device), out[b * region + i] for i < counts[b] are its claimed slots less
 * offs[b], ascending; counts[b] their number (at most region are written).
 * The list holds min(*n_dev, cap) entries; cap <= PLX_CLAIMED_SPLIT_MAX.
 * No counterpart in the reference, whose claim writes the bucket in place:
 * it lets the merged relayout find the claimed slots without comparing DEAD
 * before and after the claim over the whole bucket. */
#define PLX_CLAIMED_SPLIT_MAX 4096
PLX_EXPORT int plx_claimed_split(int64_t cap, const int32_t* n_dev, const int32_t* list, int32_t nb,
                                 const int64_t* offs, int64_t region, int32_t* out, int32_t* counts,
                                 void* stream);

/* PIPELINE claim domains (phases.py:3040-3049): for the listed slots,
 * out[p] = level[clamp(ids[idx[p]], 0, bound - 1)], the level of each dead
 * slot's former source (n_max, count n_dev). */
PLX_EXPORT int plx_gather_level(int64_t n_max, const int32_t* n_dev, const int32_t* idx,
                                const int32_t* ids, const int32_t* level, int32_t bound, int32_t* out,
                                void* stream);

/* Occurrence of each live edge among its parallel edges (phases.py:
 * 3990-4007): sorted lists the flat slots by (src, dst, slot), dead last;
 * occ[sorted[p]] = p - (first position of that pair). */
PLX_EXPORT int plx_occurrence(int64_t n, const int32_t* sorted, const int32_t* from_id,
                              const int32_t* to_id, int32_t* occ, void* stream);

/* Small helpers of the growth pipeline: out[p] = a[idx[p]] (gather); per
 * level counts of n keys (count in n_dev, optional) and the exclusive scan
 * of those counts (count, start: nlevels each; scratch plx_scratch_ints(
 * nlevels) ints); each bucket's run of the ascending free list (bucket_off:
 * num_buckets + 1 flat offsets; free_info: start, length per bucket). */
PLX_EXPORT int plx_gather_i32(int64_t n_max, const int32_t* n_dev, const int32_t* idx,
                              const int32_t* a, int32_t* out, void* stream);
PLX_EXPORT int plx_level_counts(int64_t n, const int32_t* n_dev, const int32_t* keys, int32_t nlevels,
                                int32_t* count, int32_t* start, int32_t* scratch, void* stream);
PLX_EXPORT int plx_bucket_free(int32_t num_buckets, const int64_t* bucket_off,
                               const int32_t* free_slots, const int32_t* nfree_total,
                               int32_t* free_info, void* stream);
/* Unit lifecycle (phases.py:1148-1193, :1245-1441). A unit column list:
 * pointer, element size (4, or 1 for bool columns), default bits. */
#define PLX_MAX_UNIT_COLS 16
typedef struct plx_unit_col {
  void* ptr;
  int32_t bytes;
  uint32_t default_bits;
} plx_unit_col;

/* Masked unit writes: for r < n (count n_dev, optional), unit u = idx ? idx[r]
 * : r gets cols[k][u] = outs[k][r] (32-bit patterns; byte columns take
 * value != 0), unless skip[u] != 0 (skip optional: the PRUNED column for
 * update_unit's live mask, phases.py:1184-1190). */
PLX_EXPORT int plx_unit_write(int64_t n, const int32_t* n_dev, const int32_t* idx, const uint8_t* skip,
                              int32_t ncols, const plx_unit_col* cols, const uint32_t* const* outs,
                              void* stream);

/* prune_unit (phases.py:1245-1307): doomed[u] = selected[u] && !pruned[u] &&
 * !exempt[u]; a doomed unit's columns in cols take their defaults, PRUNED
 * is set, and doomed_count counts them. */
PLX_EXPORT int plx_unit_prune(int64_t n, const uint32_t* selected, uint8_t* pruned, const uint8_t* exempt,
                              int32_t ncols, const plx_unit_col* cols, uint8_t* doomed, int32_t* doomed_count,
                              void* stream);

/* Commits the fused forward's tombstones (build_prune_merge_phase,
 * phases.py:2447-2469) over n positions: where sink[p] is set and dead[p]
 * is not, dead[p] = 1 and stamp (optional) gets stamp_value (see
 * plx_kill_incident). */
PLX_EXPORT int plx_merge_kills(int64_t n, const uint8_t* sink, uint8_t* dead, float* stamp, float stamp_value,
                               void* stream);

/* The incident-edge kill of prune_unit: dead[p] |= doomed[from[p]] |
 * doomed[to[p]] over n positions (ids mapped through id_map when set);
 * kill_count (optional) counts the bytes turned to 1, and stamp (optional)
 * gets stamp_value at each of them (a column the caller keeps implicit while
 * an edge lives, such as a uniform Adam step count, frozen at the kill). */
PLX_EXPORT int plx_kill_incident(int64_t n, const int32_t* from_id, const int32_t* to_id, uint8_t* dead,
                                 const uint8_t* doomed, const int32_t* id_map, int32_t* kill_count,
                                 float* stamp, float stamp_value, void* stream);

/* add_unit's placement (phases.py:1376-1405): the r-th parent (parents:
 * ascending live spawning ids, *nparents) takes the r-th free slot (free:
 * ascending PRUNED ids, *nfree): its columns take their defaults, its level
 * clamp(level[parent] + offset[parent], 1, max_level), PRUNED is cleared;
 * child[r], parent[r] list the placements. flags[0] = placed count, flags[1]
 * = 1 when some parent found no slot. */
PLX_EXPORT int plx_unit_place(int64_t n_max, const int32_t* parents, const int32_t* nparents,
                              const int32_t* free_ids, const int32_t* nfree, const int32_t* offset,
                              int32_t* level, uint8_t* pruned, int32_t max_level, int32_t ncols,
                              const plx_unit_col* cols, int32_t* child, int32_t* parent, int32_t* flags,
                              void* stream);

/* topo.resort (topo.py:189-452): one Bellman-Ford round of longest-path
 * levels over the live edges: out = max(in, max over live (u -> v) of
 * in[u] + 1), then (pin_inputs) every input back to 0; changed[0] = 1 when
 * any level moved. `out` must start as a copy of `in` (plx_relax_levels
 * copies it). */
PLX_EXPORT int plx_relax_levels(int64_t n_units, int64_t n_edges, const int32_t* from_id,
                                const int32_t* to_id, const uint8_t* dead, const int32_t* level_in,
                                int32_t* level_out, const uint8_t* is_input, int32_t* changed,
                                void* stream);

/* CSR offsets from ascending row ids: start[u] = the number of keys[0, n)
 * below u, for u in [0, nlevels] (keys in [0, nlevels)); n_dev (optional)
 * holds the key count (at most n) on the device. */
PLX_EXPORT int plx_sorted_starts(int64_t n, const int32_t* n_dev, const int32_t* keys, int32_t nlevels, int32_t* start,
                                 void* stream);

/* Resort keys: key[p] = dead[p] ? sentinel : (pipeline ? 0 : level[from[p]]). */
PLX_EXPORT int plx_resort_keys(int64_t n, const int32_t* from_id, const uint8_t* dead, const int32_t* level,
                               int32_t pipeline, int32_t sentinel, int32_t* key, void* stream);

/* Column gather: dst[p] = src[idx[p]] for p < n (count n_dev, optional),
 * elements of `bytes` (1 or 4) bytes. */
PLX_EXPORT int plx_gather_col(int64_t n, const int32_t* n_dev, const int32_t* idx, const void* src, void* dst,
                              int32_t bytes, void* stream);

/* importance masks for the shortlists (phases.py:3683-3746): out[u] = imp[u]
 * where (mode 0: level[u] == b; mode 1: |level[u] - b| <= gap with the
 * direction; mode 2: always) and the unit is live, else -inf. */
PLX_EXPORT int plx_mask_importance(int32_t n, const float* imp, const int32_t* level,
                                   const uint8_t* pruned, int32_t mode, int32_t b,
                                   int32_t gap, int32_t direction, float* out, void* stream);

PLX_EXPORT const char* plx_last_error(void);
/* The tiled arena's backward tables on the device (the host build is
 * plastax_amd/_layout.py; the reference's arena has no transpose tables, its
 * resort being topo.py:303-452). One workgroup per tile sorts the tile's live
 * positions by (physical source, position) in LDS. Positions are relative to
 * the bucket; the first `live` hold its live edges, destination-sorted, with
 * physical FROM_ID src[p] (any non-negative int32 id: the sort keys are 64
 * bits); tile t is [tile_pos[t], tile_pos[t+1]) and spans at most 4096
 * positions.
 *   pass 0: ngroups[t] = the tile's (tile, source) groups, or -1 where the
 *           tile spans more than 4096 positions (its tables are then
 *           unusable; the caller reads the counts and refuses them);
 *           presence[u] += the tiles holding source u (presence zeroed by
 *           the caller).
 *   pass 1: sorted_rank[p] = rank of p in its tile's order | 0x8000 where the
 *           rank starts a group (positions past `live` are not written);
 *           per group, in (tile, source) order from grp_off[t]: g_src, g_st
 *           (first rank), g_tile; grp[grp_off[t]..] the tile's descriptors
 *           (first rank | min(length, 15) << 12), longest first, ties in
 *           source order; hl[2t] / hl[2t+1] the ranks of sources below
 *           hot_base / in [hot_base, hot_base + nhot); cnt[8t + x] the tile's
 *           other ranks whose source's finalize row is in region x
 *           (region[u], 0..7). */
typedef struct plx_tile_build_desc {
  int32_t ntiles;
  int32_t live;
  int32_t pass;
  int32_t hot_base;
  int32_t nhot;
  int32_t reserved;
  const int32_t* tile_pos;
  const int32_t* src;
  int32_t* ngroups;
  int32_t* presence;
  const int32_t* grp_off;
  const int8_t* region;
  uint16_t* sorted_rank;
  uint16_t* grp;
  int32_t* g_src;
  int32_t* g_st;
  int32_t* g_tile;
  int32_t* hl;
  int32_t* cnt;
} plx_tile_build_desc;

PLX_EXPORT int plx_tile_build(const plx_tile_build_desc* d, void* stream);

/* The cold slots of the tiled backward, for the cold groups cold[k] (group
 * indices of plx_tile_build's lists, ordered by (source, tile); count n_dev
 * or n): cold_idx[k] = off[8 t + region[src]] + c, c the group's first rank
 * less the tile's hot ranks before it; cold_sb[k] = sb_of_tile[t]. */
PLX_EXPORT int plx_cold_slots(int64_t n, const int32_t* n_dev, const int32_t* cold, const int32_t* g_src,
                              const int32_t* g_st, const int32_t* g_tile, const int32_t* hl, const int32_t* off,
                              const int8_t* region, const int32_t* sb_of_tile, int32_t* cold_idx,
                              uint16_t* cold_sb, void* stream);

/* The churn layout's incremental rebuild (plastax_amd/_churn.py
 * ChurnArena.merged): after a growth step the live edges are the previous
 * layout's survivors, still in (destination, slot) order, plus the slots the
 * claim filled; merging the two sorted lists gives the order a full rebuild
 * (the reference's resort, topo.py:303-452, a stable sort of every live
 * slot) would give, for the cost of one pass over the columns. */

/* dst[slot[pos[i]]] = src[pos[i]] for i < n (count n_dev, optional),
 * elements of `bytes` (1 or 4) bytes; slot values outside [0, dst_len) are
 * skipped: copies the positions listed in pos (the edges killed since the
 * layout) back into their logical slots. */
PLX_EXPORT int plx_copy_to_slots(int64_t n, const int32_t* n_dev, const int32_t* pos, const int32_t* slot,
                                 const void* src, void* dst, int64_t dst_len, int32_t bytes, void* stream);

/* One side of a merge: n elements whose ids (in [0, id_limit)) are listed
 * in ascending (key1[id], key2[id]) order, keys compared as uint32; key2
 * null means the id itself. map (optional, id_limit entries) receives each
 * element's merged rank plus the merge's offset. */
typedef struct plx_merge_side {
  int64_t n;
  int64_t id_limit;
  const int32_t* ids;
  const int32_t* key1;
  const int32_t* key2;
  int32_t* map;
  const int32_t* n_dev; /* optional: the element count (at most n) on the device */
} plx_merge_side;

/* Merges a and b (a first where keys are equal): order[r] (optional,
 * a.n + b.n entries) is a's id at merged rank r, or -1 - j for b's j-th
 * element. One thread per element of a searches b; b is meant to be the
 * short side (the claimed slots), each of its elements written by the
 * thread of the a element it precedes. */
typedef struct plx_merge_desc {
  plx_merge_side a;
  plx_merge_side b;
  int64_t offset;
  int32_t* order;
} plx_merge_desc;

PLX_EXPORT int plx_merge_index(const plx_merge_desc* d, void* stream);

/* out[r] = a[order[r]] where order[r] >= 0, else b[b_ids[j]] (b null: the
 * id b_ids[j] itself) for j = -1 - order[r], r < n; elements of `bytes`
 * (1 or 4) bytes; a has a_limit entries, b b_limit, b_ids nb. With n_dev
 * (optional) only the first *n_dev ranks are gathered (at most n) and ranks
 * [*n_dev, n) get each column's `fill` bits. */
typedef struct plx_merge_col {
  const void* a;
  const void* b;
  void* out;
  int32_t bytes;
  uint32_t fill;
} plx_merge_col;

#define PLX_MERGE_MAX_COLS 12

typedef struct plx_merge_gather_desc {
  int64_t n;
  const int32_t* order;
  const int32_t* b_ids;
  int64_t nb;
  int64_t a_limit;
  int64_t b_limit;
  int32_t ncols;
  int32_t reserved;
  plx_merge_col cols[PLX_MERGE_MAX_COLS];
  const int32_t* n_dev;
} plx_merge_gather_desc;

PLX_EXPORT int plx_merge_gather(const plx_merge_gather_desc* d, void* stream);

/* out[j] = map[idx[j] - off] (-1 where idx[j] - off is outside
 * [0, map_len)), live[j] = out[j] >= 0, for j < n. */
PLX_EXPORT int plx_remap_i32(int64_t n, const int32_t* idx, int64_t off, int64_t map_len, const int32_t* map,
                             int32_t* out, uint8_t* live, void* stream);

/* plx_remap_i32 for a merge's old-to-new positions, without reading the map
 * at random when the merge moved few elements: for p = idx[j] - off in
 * [0, map_len), out[j] = -1 where p is one of the dropped positions, else
 * s + c + off, with s = p less the dropped positions below it (its rank
 * among the survivors) and c the inserted elements placed before survivor
 * s; live[j] = out[j] >= 0; -1 outside [0, map_len). dropped: the dropped
 * positions (ascending, *ndropped of them, at most map_len); ins: the
 * inserted elements in merge order (*nins of them, at most ins_len),
 * new_pos[ins[i]] - off their merged ranks.
 * With more than PLX_REMAP_LDS_MAX of either, out[j] = map[p] (the map
 * plx_merge_index wrote). No counterpart in the reference, whose layout is
 * rebuilt in full. */
#define PLX_REMAP_LDS_MAX 4096
PLX_EXPORT int plx_remap_merged(int64_t n, const int32_t* idx, int64_t off, int64_t map_len, const int32_t* map,
                                const int32_t* dropped, const int32_t* ndropped, const int32_t* ins,
                                const int32_t* nins, int64_t ins_len, const int32_t* new_pos, int32_t* out,
                                uint8_t* live, void* stream);

/* counts[ids[p]] += 1 over n positions, skipping p where skip[p] (optional)
 * and ids outside [0, nbins) (integer atomics: the counts are exact). */
PLX_EXPORT int plx_count_ids(int64_t n, const int32_t* ids, const uint8_t* skip, int32_t nbins, int32_t* counts,
                             void* stream);

PLX_EXPORT int32_t plx_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PLASTAX_HIP_H_ */
