"""ctypes binding of the C ABI in include/plastax_hip.h.

The library is loaded from the package directory (built in-tree by
plastax_amd.build). There is no fallback: if the library is missing or a call
fails, the error is raised here, so a step either runs the HIP kernels or
fails loudly.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
from typing import Any

LIB_PATH = pathlib.Path(
    os.environ.get("PLASTAX_HIP_LIB")
    or pathlib.Path(__file__).resolve().parent / "libplastax_hip.so"
)

ABI_VERSION = 28  # plx_abi_version() of the library these mirrors describe

PLX_MAX_INSTR = 48
PLX_MAX_CONST = 32
PLX_MAX_FIELDS = 8
PLX_MAX_OUTS = 4
PLX_MAX_TBL = 8192
PLX_MAX_SINSTR = 160
PLX_MAX_SCONST = 32
PLX_MAX_SFIELDS = 8
PLX_MAX_SOUTS = 8
PLX_MAX_GROW_COLS = 16
PLX_SITE_ID_COLUMN = 0x100
PLX_PROBE_LDS = 0
PLX_PROBE_L2 = 1
PLX_MAX_UNIT_COLS = 16

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p


class PlxError(RuntimeError):
    """A C-ABI call returned an error code."""


class plx_program(ctypes.Structure):
    _fields_ = [
        ("ninstr", c_i32),
        ("nout", c_i32),
        ("nfields", c_i32),
        ("fixed_mask", c_i32),
        ("code", c_i32 * (4 * PLX_MAX_INSTR)),
        ("consts", c_f32 * PLX_MAX_CONST),
        ("fields", c_vp * PLX_MAX_FIELDS),
        ("outs", c_vp * PLX_MAX_OUTS),
    ]


class plx_finalize(ctypes.Structure):
    _fields_ = [
        ("level", c_vp),
        ("is_input", c_vp),
        ("pruned", c_vp),
        ("fin_level", c_i32),
        ("skip_inputs", c_i32),
    ]


PLX_MOW_FIRST = 0
PLX_MOW_ADD = 1
PLX_MOW_APPLY = 2

PLX_MAP_W_CONST = 1
PLX_MAP_X_CONST = 2


class plx_map(ctypes.Structure):
    _fields_ = [("flags", c_i32), ("w", c_f32), ("x", c_f32), ("reserved", c_i32)]


class plx_forward_desc(ctypes.Structure):
    _fields_ = [
        ("nrows", c_i32),
        ("monoid", c_i32),
        ("tbl_base", c_i32),
        ("tbl_len", c_i32),
        ("row_unit", c_vp),
        ("row_ptr", c_vp),
        ("src", c_vp),
        ("weight", c_vp),
        ("dead", c_vp),
        ("x", c_vp),
        ("acc", c_vp),
        ("fin", plx_finalize),
        ("apply", plx_program),
        ("map", plx_map),
        ("prune_prog", c_vp),
        ("prune_sink", c_vp),
        ("prune_slot", c_vp),
        ("ids_logical", c_vp),
        ("ids_physical", c_vp),
        ("prune_base", c_i64),
        ("num_units", c_i32),
        ("reserved", c_i32),
    ]


class plx_tile_desc(ctypes.Structure):
    _fields_ = [
        ("base", c_i64),
        ("end", c_i64),
        ("tile_size", c_i32),
        ("ntiles", c_i32),
        ("nsuper", c_i32),
        ("monoid", c_i32),
        ("fold", c_i32),
        ("update", c_i32),
        ("nhot", c_i32),
        ("rule", c_i32),
        ("pow_table_len", c_i32),
        ("tbl_base", c_i32),
        ("tbl_len", c_i32),
        ("hot_base", c_i32),
        ("live_end", c_i64),
        ("step_mode", c_i32),
        ("step_t", c_f32),
        ("tile_pos", c_vp),
        ("super_tile", c_vp),
        ("tile_info", c_vp),
        ("grp_off", c_vp),
        ("grp", c_vp),
        ("sorted_rank", c_vp),
        ("hot_sb", c_vp),
        ("cold_partial", c_vp),
        ("src", c_vp),
        ("dst", c_vp),
        ("dead", c_vp),
        ("weight", c_vp),
        ("s0", c_vp),
        ("s1", c_vp),
        ("s2", c_vp),
        ("g", c_vp),
        ("dst8", c_vp),
        ("blk_dst0", c_vp),
        ("gfield", c_vp),
        ("act", c_vp),
        ("pow_table", c_vp),
        ("p", c_f32 * 8),
        ("map", plx_map),
    ]


class plx_partials_desc(ctypes.Structure):
    _fields_ = [
        ("nrows", c_i32),
        ("monoid", c_i32),
        ("nsuper", c_i32),
        ("nhot", c_i32),
        ("nparts", c_i32),
        ("reserved", c_i32),
        ("part_rows", c_vp),
        ("row_unit", c_vp),
        ("row_hot", c_vp),
        ("row_cold", c_vp),
        ("hot_sb", c_vp),
        ("cold_partial", c_vp),
        ("cold_sb", c_vp),
        ("cold_idx", c_vp),
        ("acc", c_vp),
        ("fin", plx_finalize),
        ("apply", plx_program),
        ("part_info", c_vp),
    ]


class plx_update_desc(ctypes.Structure):
    _fields_ = [
        ("n", c_i64),
        ("rule", c_i32),
        ("pow_table_len", c_i32),
        ("tbl_base", c_i32),
        ("tbl_len", c_i32),
        ("live_end", c_i64),
        ("step_mode", c_i32),
        ("step_t", c_f32),
        ("src", c_vp),
        ("dst", c_vp),
        ("dead", c_vp),
        ("weight", c_vp),
        ("s0", c_vp),
        ("s1", c_vp),
        ("s2", c_vp),
        ("gfield", c_vp),
        ("act", c_vp),
        ("pow_table", c_vp),
        ("dst8", c_vp),
        ("blk_dst0", c_vp),
        ("p", c_f32 * 8),
    ]


class plx_bwd_batch_desc(ctypes.Structure):
    _fields_ = [
        ("nrows", c_i32),
        ("monoid", c_i32),
        ("batch", c_i32),
        ("reserved", c_i32),
        ("row_unit", c_vp),
        ("row_ptr", c_vp),
        ("dst", c_vp),
        ("weight", c_vp),
        ("live", c_vp),
        ("g", c_vp),
        ("acc", c_vp),
        ("fin", plx_finalize),
        ("apply", plx_program),
        ("map", plx_map),
    ]


class plx_batch_tiles(ctypes.Structure):
    _fields_ = [
        ("ntiles", c_i32),
        ("num_units", c_i32),
        ("tile_off", c_vp),
        ("tile_base", c_vp),
        ("pos", c_vp),
        ("loc", c_vp),
    ]


class plx_site_prog(ctypes.Structure):
    _fields_ = [
        ("ninstr", c_i32),
        ("nout", c_i32),
        ("reserved", c_i32 * 2),
        ("code", c_i32 * (4 * PLX_MAX_SINSTR)),
        ("consts", ctypes.c_uint32 * PLX_MAX_SCONST),
        ("ufields", c_vp * PLX_MAX_SFIELDS),
        ("cfields", c_vp * PLX_MAX_SFIELDS),
        ("ubytes", c_i32 * PLX_MAX_SFIELDS),
        ("cbytes", c_i32 * PLX_MAX_SFIELDS),
    ]


class plx_site_desc(ctypes.Structure):
    _fields_ = [
        ("prog", plx_site_prog),
        ("n", c_i64),
        ("kind", c_i32),
        ("per", c_i32),
        ("num_units", c_i32),
        ("step", c_i32),
        ("net_seed", ctypes.c_uint64),
        ("list_a", c_vp),
        ("list_b", c_vp),
        ("from_id", c_vp),
        ("to_id", c_vp),
        ("occ", c_vp),
        ("n_dev", c_vp),
        ("outs", c_vp * PLX_MAX_SOUTS),
        ("or_into", c_vp),
        ("kill_count", c_vp),
        ("site_ids", c_vp),
        ("ids_logical", c_vp),
        ("ids_physical", c_vp),
        ("batch", c_i32),
        ("sample", c_i32),
        ("stamp", c_vp),
        ("stamp_value", ctypes.c_float),
    ]


class plx_tile_build_desc(ctypes.Structure):
    _fields_ = [
        ("ntiles", c_i32),
        ("live", c_i32),
        ("pass_", c_i32),
        ("hot_base", c_i32),
        ("nhot", c_i32),
        ("reserved", c_i32),
        ("tile_pos", c_vp),
        ("src", c_vp),
        ("ngroups", c_vp),
        ("presence", c_vp),
        ("grp_off", c_vp),
        ("region", c_vp),
        ("sorted_rank", c_vp),
        ("grp", c_vp),
        ("g_src", c_vp),
        ("g_st", c_vp),
        ("g_tile", c_vp),
        ("hl", c_vp),
        ("cnt", c_vp),
    ]


class plx_merge_side(ctypes.Structure):
    _fields_ = [
        ("n", c_i64),
        ("id_limit", c_i64),
        ("ids", c_vp),
        ("key1", c_vp),
        ("key2", c_vp),
        ("map", c_vp),
        ("n_dev", c_vp),
    ]


class plx_merge_desc(ctypes.Structure):
    _fields_ = [
        ("a", plx_merge_side),
        ("b", plx_merge_side),
        ("offset", c_i64),
        ("order", c_vp),
    ]


PLX_MERGE_MAX_COLS = 12
PLX_CLAIMED_SPLIT_MAX = 4096
PLX_REMAP_LDS_MAX = 4096


class plx_merge_col(ctypes.Structure):
    _fields_ = [
        ("a", c_vp),
        ("b", c_vp),
        ("out", c_vp),
        ("bytes", c_i32),
        ("fill", ctypes.c_uint32),
    ]


class plx_merge_gather_desc(ctypes.Structure):
    _fields_ = [
        ("n", c_i64),
        ("order", c_vp),
        ("b_ids", c_vp),
        ("nb", c_i64),
        ("a_limit", c_i64),
        ("b_limit", c_i64),
        ("ncols", c_i32),
        ("reserved", c_i32),
        ("cols", plx_merge_col * PLX_MERGE_MAX_COLS),
        ("n_dev", c_vp),
    ]


class plx_gen_fold_desc(ctypes.Structure):
    _fields_ = [
        ("prog", plx_site_prog),
        ("nrows", c_i32),
        ("ncomp", c_i32),
        ("backward", c_i32),
        ("num_units", c_i32),
        ("monoid", c_i32 * 8),
        ("identity", ctypes.c_float * 8),
        ("row_unit", c_vp),
        ("row_ptr", c_vp),
        ("entry_pos", c_vp),
        ("from_id", c_vp),
        ("to_id", c_vp),
        ("dead", c_vp),
        ("base", c_i64),
        ("slot", c_vp),
        ("ids_logical", c_vp),
        ("ids_physical", c_vp),
        ("acc", c_vp * 8),
        ("batch", c_i32),
        ("reserved", c_i32),
    ]


class plx_sort_key(ctypes.Structure):
    _fields_ = [("kind", c_i32), ("bits", c_i32), ("bound", c_i32), ("reserved", c_i32), ("a", c_vp), ("b", c_vp)]


class plx_sort_desc(ctypes.Structure):
    _fields_ = [
        ("n_max", c_i64),
        ("n_dev", c_vp),
        ("nkeys", c_i32),
        ("reserved", c_i32),
        ("keys", plx_sort_key * 6),
        ("vals", c_vp),
        ("keys_buf", c_vp),
        ("keys_alt", c_vp),
        ("vals_alt", c_vp),
        ("hist", c_vp),
    ]


class plx_grow_filter_desc(ctypes.Structure):
    _fields_ = [
        ("n", c_i64),
        ("grid_sq", c_i64),
        ("num_units", c_i32),
        ("num_buckets", c_i32),
        ("pipeline", c_i32),
        ("max_level_gap", c_i32),
        ("direction", c_i32),
        ("allow_self_loops", c_i32),
        ("check_range", c_i32),
        ("per", c_i32),
        ("src", c_vp),
        ("dst", c_vp),
        ("score", c_vp),
        ("level", c_vp),
        ("pruned", c_vp),
        ("proposer_idx", c_vp),
        ("proposer_dead", c_vp),
        ("nlive", c_i64),
        ("nlive_dev", c_vp),
        ("live_idx", c_vp),
        ("live_bucket", c_vp),
        ("live_src", c_vp),
        ("live_dst", c_vp),
    ]


class plx_grow_col(ctypes.Structure):
    _fields_ = [
        ("ptr", c_vp),
        ("bytes", c_i32),
        ("init_slot", c_i32),
        ("default_bits", ctypes.c_uint32),
        ("reserved", c_i32),
    ]


class plx_grow_claim_desc(ctypes.Structure):
    _fields_ = [
        ("n_max", c_i64),
        ("n_dev", c_vp),
        ("winners", c_vp),
        ("src", c_vp),
        ("dst", c_vp),
        ("score", c_vp),
        ("level", c_vp),
        ("pipeline", c_i32),
        ("num_buckets", c_i32),
        ("num_levels", c_i32),
        ("has_threshold", c_i32),
        ("threshold", c_f32),
        ("max_new_per_step", c_i32),
        ("capacity", c_i64),
        ("tail_start", c_i64),
        ("free_slots", c_vp),
        ("free_info", c_vp),
        ("own_slots", c_vp),
        ("own_start", c_vp),
        ("own_count", c_vp),
        ("from_id", c_vp),
        ("to_id", c_vp),
        ("dead", c_vp),
        ("ncols", c_i32),
        ("reserved", c_i32),
        ("cols", plx_grow_col * PLX_MAX_GROW_COLS),
        ("init_out", c_vp * PLX_MAX_SOUTS),
        ("flags", c_vp),
        ("scratch", c_vp),
        ("growable_in", c_vp),
        ("dropped_out", c_vp),
        ("tail_dev", c_vp),
        ("claimed_out", c_vp),
        ("claimed_n", c_vp),
        ("claimed_cap", c_i64),
    ]



class plx_unit_col(ctypes.Structure):
    _fields_ = [("ptr", c_vp), ("bytes", c_i32), ("default_bits", ctypes.c_uint32)]


_SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "plx_forward_bucket": (c_i32, [ctypes.POINTER(plx_forward_desc), c_vp]),
    "plx_backward_tiles": (c_i32, [ctypes.POINTER(plx_tile_desc), c_vp]),
    "plx_backward_partials": (c_i32, [ctypes.POINTER(plx_partials_desc), c_vp]),
    "plx_site_compile": (c_i32, [ctypes.POINTER(plx_site_desc), ctypes.c_char_p, ctypes.c_char_p,
                                 ctypes.POINTER(c_vp)]),
    "plx_site_eval_compiled": (c_i32, [c_vp, ctypes.POINTER(plx_site_desc), c_vp]),
    "plx_forward_prune_compile": (c_i32, [ctypes.POINTER(plx_site_desc), c_i32, ctypes.c_char_p, ctypes.c_char_p,
                                          ctypes.POINTER(c_vp)]),
    "plx_forward_bucket_compiled": (c_i32, [c_vp, ctypes.POINTER(plx_forward_desc), c_vp]),
    "plx_roof_probe": (c_i32, [c_i32, c_i32, c_vp, c_i64, c_vp, ctypes.POINTER(ctypes.c_double),
                               ctypes.POINTER(ctypes.c_float), c_vp]),
    "plx_update_conn": (c_i32, [ctypes.POINTER(plx_update_desc), c_vp]),
    "plx_scatter_f32": (c_i32, [c_i32, c_vp, c_vp, c_vp, c_vp]),
    "plx_loss_elementwise": (
        c_i32,
        [c_i32, c_vp, c_vp, ctypes.POINTER(plx_program), c_vp, c_vp, c_vp, c_vp],
    ),
    "plx_loss_softmax_ce": (c_i32, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_fill_f32": (c_i32, [c_i64, c_f32, c_vp, c_vp]),
    "plx_forward_batch": (c_i32, [ctypes.POINTER(plx_forward_desc), c_i32, c_vp]),
    "plx_backward_batch": (c_i32, [ctypes.POINTER(plx_bwd_batch_desc), c_vp]),
    "plx_update_batch": (c_i32, [ctypes.POINTER(plx_update_desc), c_i32, c_vp]),
    "plx_update_batch_tiles": (c_i32, [ctypes.POINTER(plx_update_desc), ctypes.POINTER(plx_batch_tiles), c_i32, c_vp]),
    "plx_gather_edges": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_backward_lists": (c_i32, [ctypes.POINTER(plx_bwd_batch_desc), c_vp]),
    "plx_loss_elementwise_batch": (
        c_i32,
        [c_i32, c_vp, c_vp, ctypes.POINTER(plx_program), c_vp, c_vp, c_vp, c_i32, c_vp],
    ),
    "plx_loss_softmax_ce_batch": (c_i32, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp]),
    "plx_batch_mean": (c_i32, [c_i32, c_vp, c_vp, c_vp]),
    "plx_reduce_batch": (c_i32, [c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "plx_philox32": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp]),
    "plx_eval_math": (c_i32, [c_i32, c_i64, c_vp, c_vp, c_vp, c_vp]),
    "plx_last_error": (ctypes.c_char_p, []),
    "plx_abi_version": (c_i32, []),
    "plx_struct_sizes": (c_i32, [ctypes.POINTER(c_i64), c_i32]),
    "plx_site_eval": (c_i32, [ctypes.POINTER(plx_site_desc), c_vp]),
    "plx_mean_of_writes": (c_i32, [c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "plx_compact": (c_i32, [c_i64, c_vp, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_scan_i32": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_scratch_ints": (c_i64, [c_i64]),
    "plx_compact_noalloc": (c_i32, [c_i64, c_vp, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "plx_sort": (c_i32, [ctypes.POINTER(plx_sort_desc), c_vp]),
    "plx_grow_filter": (c_i32, [ctypes.POINTER(plx_grow_filter_desc), c_vp]),
    "plx_grow_mark_repeats": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_grow_select": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_i32, c_i64, c_i32, c_vp, c_vp, c_vp]),
    "plx_grow_claim": (c_i32, [ctypes.POINTER(plx_grow_claim_desc), c_vp]),
    "plx_gather_level": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp]),
    "plx_occurrence": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_gather_i32": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_level_counts": (c_i32, [c_i64, c_vp, c_vp, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "plx_bucket_free": (c_i32, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_mask_importance": (c_i32, [c_i32, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp]),
    "plx_relax_levels": (c_i32, [c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_resort_keys": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_i32, c_i32, c_vp, c_vp]),
    "plx_gather_col": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp]),
    "plx_sorted_starts": (c_i32, [c_i64, c_vp, c_vp, c_i32, c_vp, c_vp]),
    "plx_unit_write": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp, c_vp]),
    "plx_unit_prune": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "plx_tile_build": (c_i32, [ctypes.POINTER(plx_tile_build_desc), c_vp]),
    "plx_cold_slots": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "plx_count_ids": (c_i32, [c_i64, c_vp, c_vp, c_i32, c_vp, c_vp]),
    "plx_batch_tile_limits": (c_i32, [c_vp, c_vp]),
    "plx_gen_fold": (c_i32, [ctypes.POINTER(plx_gen_fold_desc), c_vp]),
    "plx_copy_to_slots": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_vp]),
    "plx_merge_index": (c_i32, [ctypes.POINTER(plx_merge_desc), c_vp]),
    "plx_merge_gather": (c_i32, [ctypes.POINTER(plx_merge_gather_desc), c_vp]),
    "plx_remap_i32": (c_i32, [c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp]),
    "plx_claimed_split": (c_i32, [c_i64, c_vp, c_vp, c_i32, c_vp, c_i64, c_vp, c_vp, c_vp]),
    "plx_remap_merged": (c_i32, [c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp,
                                 c_vp]),
    "plx_merge_kills": (c_i32, [c_i64, c_vp, c_vp, c_vp, ctypes.c_float, c_vp]),
    "plx_kill_incident": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, ctypes.c_float, c_vp]),
    "plx_unit_place": (c_i32, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp,
                               c_vp]),
}

# Entry points the header declares (checked by the CPU test suite).
EXPORTED = tuple(_SIGNATURES)

STRUCTS = (
    plx_program,
    plx_finalize,
    plx_forward_desc,
    plx_tile_desc,
    plx_partials_desc,
    plx_update_desc,
    plx_site_prog,
    plx_site_desc,
    plx_sort_key,
    plx_sort_desc,
    plx_grow_filter_desc,
    plx_grow_col,
    plx_grow_claim_desc,
    plx_unit_col,
    plx_bwd_batch_desc,
    plx_batch_tiles,
    plx_tile_build_desc,
    plx_gen_fold_desc,
    plx_merge_desc,
    plx_merge_gather_desc,
)

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the in-tree HIP library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build the HIP library with `python -m plastax_amd.build`"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.plx_abi_version() != ABI_VERSION:
        raise ImportError(
            f"{LIB_PATH} has ABI version {lib.plx_abi_version()}, expected {ABI_VERSION}: rebuild it"
        )
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raise PlxError for a non-zero return code."""
    if rc != 0:
        msg = load().plx_last_error()
        raise PlxError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")


def call(name: str, *args: Any) -> None:
    """Call an entry point and raise on error."""
    check(getattr(load(), name)(*args), name)
