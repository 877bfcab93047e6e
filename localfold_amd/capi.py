"""ctypes mirror of include/localfold.h (structs, enums, prototypes) and the library loader.

The library is localfold_amd/lib/liblocalfold.so, built in-tree by localfold_amd.build.
Loading fails loudly when it is missing: there is no fallback path.
"""
import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "liblocalfold.so"

LF_OK, LF_ERR_INVALID, LF_ERR_DEVICE, LF_ERR_MEMORY, LF_ERR_UNSUPPORTED = 0, 1, 2, 3, 4
LF_F32, LF_F16, LF_BF16, LF_INT8, LF_INT5 = 0, 1, 2, 3, 4
LF_IN_OUT, LF_OUT_IN = 0, 1
LF_OUTGOING, LF_INCOMING = 0, 1
LF_AF2, LF_AF3 = 0, 1
LF_BIAS_NONE, LF_BIAS_SEPARATE, LF_BIAS_NORMALIZED_INPUT, LF_BIAS_LOGITS = 0, 1, 2, 3
LF_TRANSITION_RELU, LF_TRANSITION_SWIGLU = 0, 1

P = C.c_void_p
FP = C.POINTER(C.c_float)


class lf_weight(C.Structure):
    _fields_ = [("dtype", C.c_int), ("layout", C.c_int), ("rows", C.c_int), ("cols", C.c_int),
                ("group", C.c_int), ("data", P), ("scales", P), ("zeros", P)]


class lf_kernel_timing(C.Structure):
    _fields_ = [("label", C.c_char * 48), ("ms", C.c_float)]


class lf_tri_mult_weights(C.Structure):
    _fields_ = [("ln_in_scale", P), ("ln_in_offset", P),
                ("ap", lf_weight), ("ag", lf_weight), ("bp", lf_weight), ("bg", lf_weight),
                ("ap_bias", P), ("ag_bias", P), ("bp_bias", P), ("bg_bias", P),
                ("ln_out_scale", P), ("ln_out_offset", P),
                ("wz", lf_weight), ("wz_bias", P), ("wg", lf_weight), ("wg_bias", P)]


class lf_tri_mult_args(C.Structure):
    _fields_ = [("direction", C.c_int), ("dialect", C.c_int), ("divide_by_length", C.c_int),
                ("length", C.c_int), ("c_z", C.c_int), ("c_hidden", C.c_int),
                ("act_dtype", C.c_int), ("z", P), ("mask", P), ("out", P), ("accumulate", C.c_int),
                ("epsilon", C.c_float), ("w", C.POINTER(lf_tri_mult_weights))]


class lf_attention_weights(C.Structure):
    _fields_ = [("norm_scale", P), ("norm_offset", P),
                ("wq", lf_weight), ("wk", lf_weight), ("wv", lf_weight), ("wg", lf_weight), ("wo", lf_weight),
                ("q_bias", P), ("g_bias", P), ("o_bias", P),
                ("pair_norm_scale", P), ("pair_norm_offset", P), ("wb", lf_weight)]


class lf_attention_args(C.Structure):
    _fields_ = [("batch", C.c_int), ("queries", C.c_int), ("channels", C.c_int), ("heads", C.c_int),
                ("head_dim", C.c_int), ("transpose", C.c_int), ("act_dtype", C.c_int), ("act", P),
                ("mask", P), ("out", P), ("accumulate", C.c_int), ("fast_variance", C.c_int),
                ("bias_mode", C.c_int), ("swap_bias", C.c_int), ("pair_dtype", C.c_int), ("pair", P),
                ("pair_channels", C.c_int), ("bias_logits", P), ("epsilon", C.c_float),
                ("w", C.POINTER(lf_attention_weights))]


class lf_transition_weights(C.Structure):
    _fields_ = [("norm_scale", P), ("norm_offset", P), ("w1", lf_weight), ("b1", P),
                ("w2", lf_weight), ("b2", P)]


class lf_transition_args(C.Structure):
    _fields_ = [("kind", C.c_int), ("rows", C.c_int), ("channels", C.c_int), ("hidden", C.c_int),
                ("act_dtype", C.c_int), ("act", P), ("out", P), ("accumulate", C.c_int),
                ("fast_variance", C.c_int), ("chunk_bytes", C.c_longlong), ("epsilon", C.c_float),
                ("w", C.POINTER(lf_transition_weights))]


class lf_opm_weights(C.Structure):
    _fields_ = [("norm_scale", P), ("norm_offset", P), ("wl", lf_weight), ("wr", lf_weight),
                ("bl", P), ("br", P), ("wo", lf_weight), ("bo", P)]


class lf_opm_args(C.Structure):
    _fields_ = [("sequences", C.c_int), ("length", C.c_int), ("c_m", C.c_int), ("c_outer", C.c_int),
                ("c_z", C.c_int), ("msa_dtype", C.c_int), ("msa", P), ("mask", P), ("pair_dtype", C.c_int),
                ("pair_in", P), ("out", P), ("accumulate", C.c_int), ("fast_variance", C.c_int),
                ("epsilon", C.c_float), ("norm_epsilon", C.c_float), ("w", C.POINTER(lf_opm_weights))]


class lf_global_attention_weights(C.Structure):
    _fields_ = [("norm_scale", P), ("norm_offset", P), ("wq", lf_weight), ("wk", lf_weight), ("wv", lf_weight),
                ("wg", lf_weight), ("g_bias", P), ("wo", lf_weight), ("o_bias", P)]


class lf_global_attention_args(C.Structure):
    _fields_ = [("sequences", C.c_int), ("length", C.c_int), ("channels", C.c_int), ("heads", C.c_int),
                ("head_dim", C.c_int), ("act_dtype", C.c_int), ("act", P), ("mask", P), ("out", P),
                ("accumulate", C.c_int), ("epsilon", C.c_float), ("w", C.POINTER(lf_global_attention_weights))]


class lf_evoformer_weights(C.Structure):
    _fields_ = [("row_attention", lf_attention_weights), ("row_heads", C.c_int),
                ("column_attention", lf_attention_weights), ("column_heads", C.c_int),
                ("msa_transition", lf_transition_weights), ("outer_product_mean", lf_opm_weights),
                ("tri_out", lf_tri_mult_weights), ("tri_in", lf_tri_mult_weights),
                ("tri_att_start", lf_attention_weights), ("tri_att_start_heads", C.c_int),
                ("tri_att_end", lf_attention_weights), ("tri_att_end_heads", C.c_int),
                ("pair_transition", lf_transition_weights)]


class lf_evoformer_block_args(C.Structure):
    _fields_ = [("sequences", C.c_int), ("length", C.c_int), ("c_m", C.c_int), ("c_z", C.c_int),
                ("c_outer", C.c_int), ("tri_hidden", C.c_int), ("msa_hidden", C.c_int), ("pair_hidden", C.c_int),
                ("msa_dtype", C.c_int), ("msa", P), ("pair_dtype", C.c_int), ("pair", P),
                ("msa_mask", P), ("pair_mask", P), ("epsilon", C.c_float),
                ("w", C.POINTER(lf_evoformer_weights))]


class lf_extra_msa_weights(C.Structure):
    _fields_ = [("base", lf_evoformer_weights), ("column_global", lf_global_attention_weights),
                ("column_global_heads", C.c_int)]


class lf_pairformer_weights(C.Structure):
    _fields_ = [("tri_out", lf_tri_mult_weights), ("tri_in", lf_tri_mult_weights),
                ("att_start", lf_attention_weights), ("att_end", lf_attention_weights), ("pair_heads", C.c_int),
                ("pair_transition", lf_transition_weights),
                ("single_logits_norm_scale", P), ("single_logits_norm_offset", P),
                ("single_logits_projection", lf_weight),
                ("single_attention", lf_attention_weights), ("single_heads", C.c_int),
                ("single_head_dim", C.c_int), ("single_transition", lf_transition_weights)]


class lf_pairformer_block_args(C.Structure):
    _fields_ = [("tokens", C.c_int), ("c_z", C.c_int), ("c_s", C.c_int),
                ("swap_transposed_bias", C.c_int), ("divide_by_length", C.c_int),
                ("pair_dtype", C.c_int), ("pair", P), ("single_dtype", C.c_int), ("single", P),
                ("pair_mask", P), ("seq_mask", P), ("transition_chunk_bytes", C.c_longlong),
                ("epsilon", C.c_float), ("w", C.POINTER(lf_pairformer_weights))]


class lf_input_embedder_weights(C.Structure):
    _fields_ = [(n, P) for n in ("preprocess_1d_w", "preprocess_1d_b", "preprocess_msa_w", "preprocess_msa_b",
                                 "left_w", "left_b", "right_w", "right_b", "prev_pos_w", "prev_pos_b",
                                 "prev_msa_norm_scale", "prev_msa_norm_offset", "prev_pair_norm_scale",
                                 "prev_pair_norm_offset", "relpos_w", "relpos_b", "extra_w", "extra_b")]


class lf_input_embedder_args(C.Structure):
    _fields_ = ([(n, C.c_int) for n in ("length", "msa_sequences", "extra_sequences", "target_channels",
                                        "msa_feature_channels", "c_m", "c_z", "c_e")]
                + [(n, P) for n in ("target_feat", "msa_feat", "extra_msa", "extra_has_deletion",
                                    "extra_deletion_value", "residue_index", "aatype", "prev_msa_first_row",
                                    "prev_pair", "prev_positions")]
                + [("msa_dtype", C.c_int), ("msa", P), ("pair_dtype", C.c_int), ("pair", P),
                   ("extra_dtype", C.c_int), ("extra", P), ("epsilon", C.c_float),
                   ("w", C.POINTER(lf_input_embedder_weights))])


class lf_af2_recycle_args(C.Structure):
    _fields_ = [("embed", lf_input_embedder_args),
                ("extra", lf_evoformer_block_args), ("extra_blocks", C.POINTER(lf_extra_msa_weights)),
                ("extra_block_count", C.c_int),
                ("main", lf_evoformer_block_args), ("main_blocks", C.POINTER(lf_evoformer_weights)),
                ("main_block_count", C.c_int)]


class lf_pair_averaging_weights(C.Structure):
    _fields_ = [("act_norm_scale", P), ("act_norm_offset", P), ("pair_norm_scale", P), ("pair_norm_offset", P),
                ("pair_logits", lf_weight), ("wv", lf_weight), ("wg", lf_weight), ("wo", lf_weight)]


class lf_pair_averaging_args(C.Structure):
    _fields_ = [("sequences", C.c_int), ("tokens", C.c_int), ("c_m", C.c_int), ("c_z", C.c_int),
                ("heads", C.c_int), ("head_dim", C.c_int), ("msa_dtype", C.c_int), ("msa", P), ("msa_mask", P),
                ("pair_dtype", C.c_int), ("pair", P), ("out", P), ("accumulate", C.c_int),
                ("epsilon", C.c_float), ("w", C.POINTER(lf_pair_averaging_weights))]


class lf_msa_module_weights(C.Structure):
    _fields_ = [("outer_product_mean", lf_opm_weights), ("c_outer", C.c_int),
                ("msa_attention", lf_pair_averaging_weights), ("msa_heads", C.c_int), ("msa_head_dim", C.c_int),
                ("msa_transition", lf_transition_weights), ("pair", lf_pairformer_weights)]


class lf_msa_block_args(C.Structure):
    _fields_ = [("sequences", C.c_int), ("tokens", C.c_int), ("c_m", C.c_int), ("c_z", C.c_int),
                ("msa_update_before_opm", C.c_int), ("swap_transposed_bias", C.c_int),
                ("divide_by_length", C.c_int), ("msa_dtype", C.c_int), ("msa", P), ("pair_dtype", C.c_int),
                ("pair", P), ("msa_mask", P), ("pair_mask", P), ("transition_chunk_bytes", C.c_longlong),
                ("epsilon", C.c_float), ("w", C.POINTER(lf_msa_module_weights))]


# (name, restype, argtypes) for every function include/localfold.h declares.
PROTOTYPES = [
    ("lf_context_create", P, [C.c_int]),
    ("lf_context_destroy", None, [P]),
    ("lf_context_set_stream", C.c_int, [P, P]),
    ("lf_last_error", C.c_char_p, []),
    ("lf_version", C.c_char_p, []),
    ("lf_malloc", C.c_int, [P, C.c_size_t, C.POINTER(P)]),
    ("lf_free", C.c_int, [P, P]),
    ("lf_memcpy_htod", C.c_int, [P, P, P, C.c_size_t]),
    ("lf_memcpy_dtoh", C.c_int, [P, P, P, C.c_size_t]),
    ("lf_memset", C.c_int, [P, P, C.c_int, C.c_size_t]),
    ("lf_synchronize", C.c_int, [P]),
    ("lf_memory_stats", C.c_int, [P, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    ("lf_profile_enable", C.c_int, [P, C.c_int]),
    ("lf_profile_read", C.c_int, [P, C.POINTER(lf_kernel_timing), C.c_int]),
    ("lf_tri_mult", C.c_int, [P, C.POINTER(lf_tri_mult_args)]),
    ("lf_tri_mult_noalloc", C.c_int, [P, C.POINTER(lf_tri_mult_args)]),
    ("lf_attention", C.c_int, [P, C.POINTER(lf_attention_args)]),
    ("lf_transition", C.c_int, [P, C.POINTER(lf_transition_args)]),
    ("lf_outer_product_mean", C.c_int, [P, C.POINTER(lf_opm_args)]),
    ("lf_global_column_attention", C.c_int, [P, C.POINTER(lf_global_attention_args)]),
    ("lf_evoformer_block", C.c_int, [P, C.POINTER(lf_evoformer_block_args)]),
    ("lf_extra_msa_block", C.c_int, [P, C.POINTER(lf_evoformer_block_args), C.POINTER(lf_extra_msa_weights)]),
    ("lf_extra_msa_stack", C.c_int, [P, C.POINTER(lf_evoformer_block_args), C.POINTER(lf_extra_msa_weights), C.c_int]),
    ("lf_evoformer_stack", C.c_int, [P, C.POINTER(lf_evoformer_block_args), C.POINTER(lf_evoformer_weights), C.c_int]),
    ("lf_evoformer_pair_stack", C.c_int, [P, C.POINTER(lf_evoformer_block_args), C.POINTER(lf_evoformer_weights), C.c_int]),
    ("lf_pairformer_block", C.c_int, [P, C.POINTER(lf_pairformer_block_args)]),
    ("lf_input_embedder", C.c_int, [P, C.POINTER(lf_input_embedder_args)]),
    ("lf_af2_recycle", C.c_int, [P, C.POINTER(lf_af2_recycle_args)]),
    ("lf_msa_pair_weighted_averaging", C.c_int, [P, C.POINTER(lf_pair_averaging_args)]),
    ("lf_msa_module_block", C.c_int, [P, C.POINTER(lf_msa_block_args)]),
]

_lib = None


class LocalfoldError(RuntimeError):
    pass


def load(path: Path = None) -> C.CDLL:
    """Loads liblocalfold.so (once) and binds every prototype.  Raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path or os.environ.get("LOCALFOLD_LIB", LIB_PATH))
    if not p.exists():
        raise LocalfoldError(f"{p} is missing: build it with `python -m localfold_amd.build` "
                             "(there is no CPU fallback)")
    lib = C.CDLL(str(p))
    for name, res, args in PROTOTYPES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != LF_OK:
        msg = load().lf_last_error()
        raise LocalfoldError(f"localfold error {rc}: {msg.decode() if msg else ''}")
