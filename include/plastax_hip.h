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
 * INTEGRATION.md shows the jax.ffi / XLA custom-call binding.
 */
#ifndef PLASTAX_HIP_H_
#define PLASTAX_HIP_H_

#include <stdint.h>

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
 * (it travels in the kernel argument segment). */
typedef struct plx_program {
  int32_t ninstr;
  int32_t nout;
  int32_t nfields;
  int32_t reserved;
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

/* One bucket of the forward pass: _accumulate_into + _apply_masked
 * (sweep.py:113-230, phases.py:972-1015) for a linear map
 * weight * x[from] (phases.py:535-556). Rows are destination units in a CSR
 * over the physical (destination-sorted) positions; each row is folded in slot
 * order, combined into acc, and finalized rows apply `apply` and reset acc.
 * `dead` may be null when no row range holds a tombstone. */
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
 * group, in physical order, into a tile partial: a hot source's tile partial
 * is folded, in tile order, into its superblock sum, stored at
 * hot_sb[superblock * nhot + h] (the identity where the source is absent);
 * the other sources' tile partials are stored in their slot of the
 * cold_partial array (group target -1-h or the cold slot; a tile's cold slots
 * are consecutive, in its group order). With
 * `update`, the same pass applies the update rule (see plx_update_desc for
 * p[] and the state columns) with grad = gfield[dst] * act[src] and stores
 * the new weight and state; dead edges keep theirs. Tile metadata:
 * sorted_rank[p - base] is the rank of live position p in its tile's
 * (source, position) order; grp_off[tile..tile+1] ranges the tile's groups;
 * grp_se packs a group's first rank (low 16 bits) and length (high 16
 * bits); tile_size is at most 4096. */
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
  int64_t live_end; /* with dead == null: positions >= live_end are dead   */
  int32_t step_mode; /* Adam: 0 per-edge step count s2; 1 every live edge  */
  float step_t;      /* has the step count step_t (s2 neither read nor      */
                     /* written; the caller advances step_t after the call) */
  const int32_t* tile_pos;   /* [ntiles+1] tile starts relative to base   */
  const int32_t* super_tile; /* [nsuper+1] first tile of each superblock  */
  const int32_t* grp_off;
  const uint32_t* grp_se;
  const int32_t* grp_tgt;
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
  const float* gfield;  /* the update rule's grad field                  */
  const float* act;     /* ACTIVATION                                    */
  const float* pow_table;
  float p[8];
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
  float p[8];
} plx_update_desc;

PLX_EXPORT int plx_update_conn(const plx_update_desc* d, void* stream);

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
 * 1 log, 2 tanh, 3 sigmoid, 4 sqrt, 5 Adam power b^t with b=x[i], t=y[i]). */
PLX_EXPORT int plx_eval_math(int32_t op, int64_t n, const float* x, const float* y,
                  float* out, void* stream);

/* sizeof of the descriptor structs, in the order plx_program, plx_finalize,
 * plx_forward_desc, plx_tile_desc, plx_partials_desc, plx_update_desc (for binding layers to check their mirrors). Writes
 * min(n, 6) values and returns 6. */
PLX_EXPORT int plx_struct_sizes(int64_t* out, int32_t n);

PLX_EXPORT const char* plx_last_error(void);
PLX_EXPORT int32_t plx_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PLASTAX_HIP_H_ */
