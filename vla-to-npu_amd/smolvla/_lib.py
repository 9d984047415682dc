"""ctypes binding of ``libsvla.so`` (the C-ABI declared in ``include/svla.h``).

The library is the only compute path: there is no CPU fallback.  Loading
fails loudly if the library has not been built.
"""

from __future__ import annotations

import ctypes
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libsvla.so"

_p = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_long
_f = ctypes.c_float
_d = ctypes.c_double
_fp = ctypes.POINTER(ctypes.c_float)

class ExpertLayer(ctypes.Structure):
    """``svla_expert_layer`` (include/svla.h)."""
    _fields_ = [("cross", ctypes.c_int), ("w_qkv", _p), ("w_o", _p), ("w_gu", _p),
                ("w_down", _p), ("norm1", _p), ("norm2", _p), ("cross_k", _p), ("cross_v", _p)]


class ExpertDesc(ctypes.Structure):
    """``svla_expert_desc`` (include/svla.h)."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "batch", "chunk", "hidden", "n_q_heads", "n_kv_heads", "head_dim", "inter",
        "action_dim", "n_layers", "prefix_len", "num_steps", "ld_cross")] + [
        ("rms_eps", ctypes.c_float), ("dt", ctypes.c_float),
        ("w_action_in", _p), ("b_action_in", _p), ("w_time_in_a", _p), ("time_bias", _p),
        ("w_time_out", _p), ("b_time_out", _p), ("norm_out", _p), ("w_action_out", _p),
        ("rope_cos", _p), ("rope_sin", _p), ("x_in", _p), ("x_out", _p),
        ("layers", ctypes.POINTER(ExpertLayer))]


class ExpertPlan(ctypes.Structure):
    """``svla_expert_plan`` (include/svla.h)."""
    _fields_ = [("phases", _p), ("n_phases", ctypes.c_int), ("counters", _p),
                ("counter_words", ctypes.c_long), ("status", _p), ("grid", ctypes.c_int),
                ("team_xcd", ctypes.c_int), ("team_size", ctypes.c_int),
                ("spin_limit", ctypes.c_int), ("stamps", _p)]


# name -> argtypes (all return int, except RESTYPES)
SIGNATURES = {
    "svla_version": [],
    "svla_init": [],
    "svla_rmsnorm_bf16": [_p, _i, _p, _p, _i, _i, _i, _f, _p],
    "svla_layernorm_bf16": [_p, _i, _p, _p, _p, _i, _i, _i, _f, _p],
    "svla_layernorm_blocked_bf16": [_p, _i, _p, _p, _p, _i, _i, _f, _p],
    "svla_gemm_set_tile": [_i],
    "svla_gemm_set_split": [_i],
    "svla_gemm_tile_choice": [_i, _i, _i, _i],
    "svla_linear_wide_bf16": [_p, _i, _p, _i, _p, _p, _p, _i, _p, _i, _i, _i, _i, _f, _i, _i, _p],
    "svla_slab_block_bf16": [_p, _i, _p, _i, _i, _p],
    "svla_linear_bf16": [_p, _i, _p, _i, _p, _p, _p, _i, _p, _i, _i, _i, _i, _f, _i, _i, _p, _f,
                         _p],
    "svla_linear_scratch_bf16": [_p, _i, _p, _i, _p, _p, _p, _i, _p, _i, _i, _i, _i, _f, _i, _i,
                                 _p, _f, _p],
    "svla_linear_rope_bf16": [_p, _i, _p, _i, _p, _i, _i, _i, _i, _i, _i, _p, _p, _p, _f, _p],
    "svla_linear_rope_lo_bf16": [_p, _i, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _p, _f,
                                 _p],
    "svla_linear_silu_mul_bf16": [_p, _i, _p, _i, _p, _i, _i, _i, _i, _p, _f, _p],
    "svla_patch_embed_bf16": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p],
    "svla_connector_bf16": [_p, _p, _i, _p, _i, _i, _i, _i, _i, _i, _i, _i, _p],
    "svla_action_out_euler": [_p, _i, _p, _i, _p, _i, _p, _i, _i, _i, _i, _p, _f, _f, _p],
    "svla_attention_bf16": [_p, _i, _l, _p, _i, _l, _p, _i, _l, _p, _i, _l, _i, _i, _i, _i, _i,
                            _i, _f, _i, _i, _p],
    "svla_attention_lo_bf16": [_p, _p, _i, _l, _p, _p, _i, _l, _p, _i, _l, _p, _i, _l, _i, _i, _i,
                               _i, _i, _i, _f, _i, _i, _p],
    "svla_masked_softmax_bf16": [_p, _i, _p, _i, _i, _p],
    "svla_softmax": [_p, _p, _i, _i, _i, _i, _p],
    "svla_silu_bf16": [_p, _p, _l, _p],
    "svla_gelu_bf16": [_p, _p, _l, _i, _p],
    "svla_silu_mul_bf16": [_p, _p, _p, _l, _p],
    "svla_rope": [_p, _i, _p, _i, _i, _i, _p, _p, _i, _i, _i, _p],
    "svla_rope_table": [_p, _p, _i, _i, _f, _p],
    "svla_pack_weight_bf16": [_p, _i, _p, _i, _i, _p],
    "svla_pack_gate_up_bf16": [_p, _p, _p, _i, _i, _p],
    "svla_embed_bf16": [_p, _p, _l, _i, _f, _p, _i, _l, _l, _i, _p],
    "svla_time_embedding_bf16": [_d, _i, _d, _d, _p, _p],
    "svla_f32_to_bf16": [_p, _p, _l, _p],
    "svla_image_to_bf16": [_p, _l, _i, _i, _i, _p, _i, _p],
    "svla_unary_f32": [_p, _p, _l, _i, _p],
    "svla_unary_bf16": [_p, _p, _l, _i, _p],
    "svla_add_bf16": [_p, _p, _p, _l, _p],
    "svla_row_norm": [_p, _i, _p, _p, _p, _i, _i, _i, _f, _i, _i, _i, _p],
    "svla_softmax_rows": [_p, _i, _p, _i, _i, _i, _i, _i, _i, _i, _p],
    "svla_conv_patch_f32": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p],
    "svla_expert_workspace_size": [ctypes.POINTER(ExpertDesc)],
    "svla_expert_prepare": [ctypes.POINTER(ExpertDesc), _p, _l, _i, ctypes.POINTER(ExpertPlan),
                            _p],
    "svla_expert_run": [ctypes.POINTER(ExpertPlan), _p],
    "svla_expert_status": [ctypes.POINTER(ExpertPlan), ctypes.POINTER(ctypes.c_int)],
    "svla_expert_trace_offset": [ctypes.POINTER(ExpertDesc), _i, _i],
}

RESTYPES = {"svla_expert_workspace_size": ctypes.c_long,
            "svla_expert_trace_offset": ctypes.c_long}

_LIB = None


def load(path: pathlib.Path = LIB_PATH):
    """Load and type the library (cached)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built; run `python -m smolvla.build` (or __graft_entry__.build()). "
            "There is no CPU fallback for the SmolVLA kernels.")
    lib = ctypes.CDLL(str(path))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = RESTYPES.get(name, ctypes.c_int)
    _LIB = lib
    return lib


class SvlaError(RuntimeError):
    pass


_OBSERVER = None


def set_observer(fn):
    """Install ``fn(name, args, run) -> rc`` around every ``call`` (``run()``
    makes the call), or remove it with None.  Used by the kernel census."""
    global _OBSERVER
    _OBSERVER = fn


def call(name: str, *args):
    f = getattr(load(), name)
    rc = f(*args) if _OBSERVER is None else _OBSERVER(name, args, lambda: f(*args))
    if rc != 0:
        what = ("invalid argument (shape / alignment)" if rc == -22 else
                "split needs more scratch than the static array holds" if rc == -28 else
                f"HIP error {rc}")
        raise SvlaError(f"{name}: {what}")
    return rc
