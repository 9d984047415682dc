"""PyTorch-facing wrappers over the C-ABI (device tensors in, device tensors out).

Every function launches on ``torch.cuda.current_stream()`` and returns
immediately (asynchronous, HIP-graph capturable).  Tensors must live on the
GPU; 2-D operands may be row-strided views (``stride(-1) == 1``).  Linear
weights are the packed ``[N, K]`` form made by :func:`pack_weight` /
:func:`pack_gate_up`.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

BF16 = torch.bfloat16
F32 = torch.float32

ACT = {None: 0, "none": 0, "gelu_tanh": 1, "tanh": 1, "gelu_erf": 2, "erf": 2, "silu": 3}
MASK = {"none": 0, "causal": 1, "prefix_lm": 2}



def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("smolvla ops take GPU tensors (no CPU fallback)")
    return ctypes.c_void_p(t.data_ptr())


def _addr(t):
    """Device address of a GPU tensor as an int (for ctypes struct fields)."""
    if not t.is_cuda:
        raise ValueError("smolvla ops take GPU tensors (no CPU fallback)")
    return t.data_ptr()


def _ld(t):
    if t.dim() != 2 or t.stride(-1) != 1:
        raise ValueError(f"expected a row-major 2-D view, got shape {tuple(t.shape)} "
                         f"strides {t.stride()}")
    return t.stride(0)


def _norm_args(norm):
    """``norm = (gain, eps)`` for a fused RMSNorm of the A rows, or None."""
    if norm is None:
        return None, 0.0
    w, eps = norm
    eps = torch.finfo(F32).eps if eps is None else eps
    return _ptr(w), float(eps)


# ----------------------------------------------------------------- norms ---
def rmsnorm(x, w, eps, out=None):
    eps = torch.finfo(F32).eps if eps is None else eps
    rows, cols = x.shape
    out = torch.empty(rows, cols, dtype=BF16, device=x.device) if out is None else out
    _lib.call("svla_rmsnorm_bf16", _ptr(x), _ld(x), _ptr(w), _ptr(out), _ld(out), rows, cols,
              float(eps), _stream())
    return out


def layernorm(x, g, b, eps, out=None, blocked=False):
    """LayerNorm of the rows of ``x``; ``blocked`` writes the slab-blocked
    ``[cols/32, rows, 32]`` layout (``LAYOUT_A_BLOCKED`` of :func:`linear_wide`)."""
    rows, cols = x.shape
    if blocked:
        out = torch.empty(cols // 32, rows, 32, dtype=BF16, device=x.device) if out is None else out
        _lib.call("svla_layernorm_blocked_bf16", _ptr(x), _ld(x), _ptr(g), _ptr(b), _ptr(out),
                  rows, cols, float(eps), _stream())
        return out
    out = torch.empty(rows, cols, dtype=BF16, device=x.device) if out is None else out
    _lib.call("svla_layernorm_bf16", _ptr(x), _ld(x), _ptr(g), _ptr(b), _ptr(out), _ld(out),
              rows, cols, float(eps), _stream())
    return out


# ------------------------------------------------------------------ GEMM ---
class FusedExpert:
    """The whole flow-matching action expert of one chunk in one persistent
    launch (``svla_expert_*``): prepared once for fixed buffers (weights,
    projected cross K/V, Euler state), then :meth:`run` per chunk on the
    current stream (graph-capturable)."""

    def __init__(self, cfg, expert_layers, cross, io, rope, tbias, x_state, batch, dt,
                 team_xcd=-1):
        e = cfg.expert
        # every tensor whose device address goes into the descriptor (and so
        # into the uploaded phase table) is held here for the plan's lifetime
        self._keep = []

        def addr(t):
            self._keep.append(t)
            return _addr(t)

        layers = (_lib.ExpertLayer * cfg.expert_layers)()
        ld_cross = 0                          # no cross layer: unused
        for i, P in enumerate(expert_layers):
            L = layers[i]
            L.cross = int(cfg.is_cross(i))
            L.w_qkv = addr(P["wq"] if L.cross else P["wqkv"])
            L.w_o, L.w_gu, L.w_down = addr(P["wo"]), addr(P["wgu"]), addr(P["wd"])
            L.norm1, L.norm2 = addr(P["n1"]), addr(P["n2"])
            if L.cross:
                ck, cv = cross[i]
                if ck.stride(0) != cv.stride(0):
                    raise ValueError("cross K and V need one leading dimension")
                if ld_cross and ck.stride(0) != ld_cross:
                    raise ValueError("every cross layer's K/V needs the same leading dimension")
                L.cross_k, L.cross_v = addr(ck), addr(cv)
                ld_cross = ck.stride(0)
        d = _lib.ExpertDesc()
        d.batch, d.chunk, d.hidden = batch, cfg.chunk, e.hidden
        d.n_q_heads, d.n_kv_heads, d.head_dim, d.inter = e.n_q_heads, e.n_kv_heads, e.head_dim, e.inter
        d.action_dim, d.n_layers, d.prefix_len = cfg.action_dim, cfg.expert_layers, cfg.prefix_len
        d.num_steps, d.ld_cross = cfg.num_steps, ld_cross
        from .config import resolve_eps
        d.rms_eps, d.dt = resolve_eps(e.rms_eps), float(dt)
        d.w_action_in, d.b_action_in = addr(io["w_ain"]), addr(io["b_ain"])
        d.w_time_in_a, d.time_bias = addr(io["w_tin_a"]), addr(tbias)
        d.w_time_out, d.b_time_out = addr(io["w_tout"]), addr(io["b_tout"])
        d.norm_out, d.w_action_out = addr(io["n_exp"]), addr(io["w_aout"])
        d.rope_cos, d.rope_sin = addr(rope.cos), addr(rope.sin)
        d.x_in = d.x_out = addr(x_state)
        d.layers = layers
        lib = _lib.load()
        nbytes = lib.svla_expert_workspace_size(ctypes.byref(d))
        if nbytes <= 0:
            raise ValueError("fused expert: configuration not supported")
        self.workspace = torch.empty(nbytes + 256, dtype=torch.uint8, device=x_state.device)
        base = (self.workspace.data_ptr() + 255) // 256 * 256
        self._base = base - self.workspace.data_ptr()
        self.plan = _lib.ExpertPlan()
        _lib.call("svla_expert_prepare", ctypes.byref(d), ctypes.c_void_p(base), nbytes,
                  int(team_xcd), ctypes.byref(self.plan), _stream())
        self.desc, self.layers = d, layers
        self.rows, self.hidden = batch * cfg.chunk, e.hidden
        self._frag_idx = None

    def run(self):
        _lib.call("svla_expert_run", ctypes.byref(self.plan), _stream())

    def status(self):
        st = ctypes.c_int(-1)
        _lib.call("svla_expert_status", ctypes.byref(self.plan), ctypes.byref(st))
        return st.value

    def phase_stamps(self):
        """One eager run with per-phase clock stamps (``plan.stamps``):
        ``[n_phases, 2]`` int64 ticks of the GPU's 100 MHz clock, the phase's
        start (its wait done) and its arrival, on the team's first workgroup.
        Synchronous.  A graph captured before keeps launching without stamps."""
        n = self.plan.n_phases
        buf = torch.zeros(2 * n, dtype=torch.int64, device=self.workspace.device)
        self.plan.stamps = buf.data_ptr()
        try:
            self.run()
            torch.cuda.synchronize(self.workspace.device)
        finally:
            self.plan.stamps = None
        return buf.view(n, 2).cpu()

    def phase_kinds(self):
        """Name of every phase of the launch, in order: the cross layers'
        V^T transposes (one phase), then per Euler step action-in, time-in,
        time-out, per layer norm + QKV / Q + RoPE, attention, O + residual,
        norm + gate|up + SiLU, down + residual, and action-out + Euler."""
        names = ["V^T transposes"] if any(l.cross for l in self.layers) else []
        per_layer = ("norm + {} + RoPE", "{} attention", "O + residual",
                     "norm + gate|up + SiLU", "down + residual")
        for _ in range(self.desc.num_steps):
            names += ["action in", "time in + SiLU", "time out"]
            for lay in self.layers:
                kind = "cross" if lay.cross else "self"
                qkv = "Q" if lay.cross else "QKV"
                names += [per_layer[0].format(qkv), per_layer[1].format(kind)] + list(per_layer[2:])
            names.append("action out + Euler")
        return names

    def trace(self, step, layer):
        """The activation entering expert layer ``layer`` at Euler step
        ``step`` of the last run (``layer == n_layers``: the last layer's
        output), ``[batch * chunk, hidden]`` bf16, read back from the
        workspace (``svla_expert_trace_offset``; a copy, in stream order)."""
        off = _lib.load().svla_expert_trace_offset(ctypes.byref(self.desc), int(step), int(layer))
        if off < 0:
            raise ValueError(f"no traced activation for step {step}, layer {layer}")
        M, H = self.rows, self.hidden
        nbytes = ((H + 31) // 32) * 4096          # bytes of a fragment-major [64, H] buffer
        start = self._base + off
        frag = self.workspace[start:start + nbytes].view(BF16)
        if self._frag_idx is None:
            # element (m, k) of a fragment-major buffer (svla.h)
            m = torch.arange(M, device=frag.device)[:, None]
            k = torch.arange(H, device=frag.device)[None, :]
            self._frag_idx = ((((k // 32) * 4 + m // 16) * 64 + m % 16 + 16 * ((k // 8) % 4)) * 8
                              + k % 8)
        return frag[self._frag_idx]


def init(device=None):
    """``svla_init`` on ``device`` (default: the current one): allocates the
    split-K workspace up front, so eager calls and calls captured into a HIP
    graph split long-K skinny GEMMs the same way; resolves the static scratch
    of :func:`linear_scratch`.  Once per device, before any capture."""
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        _lib.call("svla_init")


def linear(a, w, bias=None, bias_f32=None, res=None, act=None, alpha=1.0, out=None,
           out_f32=False, norm=None):
    """``epilogue(alpha * norm(a) @ w.T)``; ``w`` packed ``[N, K]``;
    ``norm=(gain, eps)`` RMS-normalises the rows of ``a`` on the fly."""
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"linear: a {tuple(a.shape)} vs packed w {tuple(w.shape)}")
    if out is None:
        out = torch.empty(M, N, dtype=F32 if out_f32 else BF16, device=a.device)
    nw, ne = _norm_args(norm)
    _lib.call("svla_linear_bf16", _ptr(a), _ld(a), _ptr(w), _ld(w), _ptr(bias), _ptr(bias_f32),
              _ptr(res), _ld(res) if res is not None else 0, _ptr(out), _ld(out), M, N, K,
              float(alpha), ACT[act], int(out_f32), nw, ne, _stream())
    return out


LAYOUT_A_BLOCKED, LAYOUT_W_BLOCKED, LAYOUT_C_BLOCKED = 1, 2, 4


def slab_block(x, out=None):
    """Row-major [rows, k] -> slab-blocked [k // 32, rows, 32] (see
    ``svla_slab_block_bf16``), returned as a flat-shaped [k // 32, rows, 32]
    tensor."""
    rows, k = x.shape
    out = torch.empty(k // 32, rows, 32, dtype=BF16, device=x.device) if out is None else out
    _lib.call("svla_slab_block_bf16", _ptr(x), _ld(x), _ptr(out), rows, k, _stream())
    return out


def unblock(xb):
    """Slab-blocked [k // 32, rows, 32] -> row-major [rows, k] (a torch view
    copy; for checks and hand-over to row-major consumers)."""
    s, rows, _ = xb.shape
    return xb.permute(1, 0, 2).reshape(rows, s * 32)


def linear_wide(a, w, m, n, k, bias=None, bias_f32=None, res=None, act=None, alpha=1.0,
                out=None, layout=0):
    """``svla_linear_wide_bf16``: the 256x256 persistent GEMM with optional
    slab-blocked A / W / C (``layout`` = OR of the LAYOUT_* flags).  Blocked
    tensors are [k // 32, rows, 32]; row-major ones are 2-D views."""
    if out is None:
        out = (torch.empty(n // 32, m, 32, dtype=BF16, device=a.device) if layout & LAYOUT_C_BLOCKED
               else torch.empty(m, n, dtype=BF16, device=a.device))
    lda = 0 if layout & LAYOUT_A_BLOCKED else _ld(a)
    ldw = 0 if layout & LAYOUT_W_BLOCKED else _ld(w)
    ldc = 0 if layout & LAYOUT_C_BLOCKED else _ld(out)
    _lib.call("svla_linear_wide_bf16", _ptr(a), lda, _ptr(w), ldw, _ptr(bias), _ptr(bias_f32),
              _ptr(res), _ld(res) if res is not None else 0, _ptr(out), ldc, m, n, k,
              float(alpha), ACT[act], int(layout), _stream())
    return out


def linear_rope(a, w, rope_cols, seq_len, cos_t, sin_t, out=None, norm=None, out_lo=None):
    """QKV projection with RoPE on the first ``rope_cols`` columns;
    ``out_lo`` (optional, the shape and row stride of ``out``) receives the
    bf16 remainder of each rotated column's fp32 value
    (``svla_linear_rope_lo_bf16``)."""
    M, K = a.shape
    N = w.shape[0]
    out = torch.empty(M, N, dtype=BF16, device=a.device) if out is None else out
    nw, ne = _norm_args(norm)
    if out_lo is not None and (out_lo.shape != out.shape or _ld(out_lo) != _ld(out)):
        raise ValueError("linear_rope: out_lo must have out's shape and row stride")
    _lib.call("svla_linear_rope_lo_bf16", _ptr(a), _ld(a), _ptr(w), _ld(w), _ptr(out),
              _ptr(out_lo), _ld(out), M, N, K, rope_cols, seq_len, _ptr(cos_t), _ptr(sin_t), nw,
              ne, _stream())
    return out


def linear_silu_mul(a, w_gu, out=None, norm=None):
    M, K = a.shape
    inter = w_gu.shape[0] // 2
    out = torch.empty(M, inter, dtype=BF16, device=a.device) if out is None else out
    nw, ne = _norm_args(norm)
    _lib.call("svla_linear_silu_mul_bf16", _ptr(a), _ld(a), _ptr(w_gu), _ld(w_gu), _ptr(out),
              _ld(out), M, inter, K, nw, ne, _stream())
    return out


def patch_embed(images, w, bias, pos, patch, out=None):
    """``images [n, C, H, H]`` bf16 contiguous; ``w [E, C*P*P]``."""
    n, C, H, W = images.shape
    E = w.shape[0]
    G = H // patch
    out = torch.empty(n * G * G, E, dtype=BF16, device=images.device) if out is None else out
    _lib.call("svla_patch_embed_bf16", _ptr(images.contiguous()), _ptr(w), _ptr(bias), _ptr(pos),
              _ptr(out), _ld(out), n, C, H, patch, E, _stream())
    return out


def connector(x, w, scale, out=None, rows_per_sample=0, sample_stride=0):
    """``x [n_img, grid*grid, hidden]`` contiguous -> ``[n_img*(grid/scale)^2, N]``
    (or remapped into a larger buffer, see ``svla_connector_bf16``)."""
    n, T, E = x.shape
    grid = int(round(math.sqrt(T)))
    N = w.shape[0]
    rows = n * (grid // scale) ** 2
    out = torch.empty(rows, N, dtype=BF16, device=x.device) if out is None else out
    if rows_per_sample:
        need = (rows // rows_per_sample - 1) * sample_stride + rows_per_sample
        if out.shape[0] < need:
            raise ValueError("connector: output buffer too small for the row remap")
    _lib.call("svla_connector_bf16", _ptr(x.contiguous()), _ptr(w), _ld(w), _ptr(out), _ld(out),
              n, grid, E, scale, N, int(rows_per_sample), int(sample_stride), _stream())
    return out


def action_out_euler(a, w, x_f32, dt, x_bf16=None, norm=None):
    M, K = a.shape
    N = w.shape[0]
    nw, ne = _norm_args(norm)
    _lib.call("svla_action_out_euler", _ptr(a), _ld(a), _ptr(w), _ld(w), _ptr(x_f32),
              _ld(x_f32), _ptr(x_bf16), _ld(x_bf16) if x_bf16 is not None else 0, M, N, K,
              nw, ne, float(dt), _stream())
    return x_f32


# ------------------------------------------------------------- attention ---
def attention(q, k, v, out, hq, hkv, mask="causal", prefix_len=0, scale=None, q_lo=None,
              k_lo=None):
    """``q [B, Sq, >=hq*64]``, ``k``/``v [B, Sk, >=hkv*64]`` (views into fused
    projection buffers are fine: row stride = ``stride(1)``), ``out [B, Sq, hq*64]``.
    ``q_lo`` / ``k_lo``: bf16 remainders of fp32 Q / K (views with q's / k's
    strides, from :func:`linear_rope`'s ``out_lo``): the scores are then taken
    on Q = q + q_lo, K = k + k_lo (``svla_attention_lo_bf16``)."""
    B, Sq = q.shape[0], q.shape[1]
    Sk = k.shape[1]
    for t in (q, k, v, out):
        if t.dim() != 3 or t.stride(-1) != 1:
            raise ValueError("attention takes [B, S, H*D] row-major views")
    for lo, hi in ((q_lo, q), (k_lo, k)):
        if lo is not None and (lo.shape != hi.shape or lo.stride() != hi.stride()):
            raise ValueError("attention: a remainder needs its operand's shape and strides")
    scale = 1.0 / math.sqrt(64) if scale is None else scale
    _lib.call("svla_attention_lo_bf16",
              _ptr(q), _ptr(q_lo), q.stride(1), q.stride(0), _ptr(k), _ptr(k_lo), k.stride(1),
              k.stride(0), _ptr(v), v.stride(1), v.stride(0), _ptr(out), out.stride(1),
              out.stride(0), B, Sq, Sk, hq, hkv, 64, float(scale), MASK[mask], int(prefix_len),
              _stream())
    return out


# ------------------------------------------------------- harness kernels ---
def masked_softmax(s, row_start, out=None):
    rows, cols = s.shape
    out = torch.empty(rows, cols, dtype=BF16, device=s.device) if out is None else out
    _lib.call("svla_masked_softmax_bf16", _ptr(s.contiguous()), int(row_start), _ptr(out), rows,
              cols, _stream())
    return out


def softmax(s, out=None, out_f32=False):
    rows, cols = s.shape
    if out is None:
        out = torch.empty(rows, cols, dtype=F32 if out_f32 else BF16, device=s.device)
    _lib.call("svla_softmax", _ptr(s.contiguous()), _ptr(out), rows, cols,
              int(s.dtype == F32), int(out.dtype == F32), _stream())
    return out


def silu(x, out=None):
    out = torch.empty_like(x) if out is None else out
    _lib.call("svla_silu_bf16", _ptr(x.contiguous()), _ptr(out), x.numel(), _stream())
    return out


def gelu(x, kind="tanh", out=None):
    out = torch.empty_like(x) if out is None else out
    _lib.call("svla_gelu_bf16", _ptr(x.contiguous()), _ptr(out), x.numel(), ACT[kind], _stream())
    return out


def silu_mul(gate, up, out=None):
    out = torch.empty_like(gate) if out is None else out
    _lib.call("svla_silu_mul_bf16", _ptr(gate.contiguous()), _ptr(up.contiguous()), _ptr(out),
              gate.numel(), _stream())
    return out


def rope(x, heads, cos_t, sin_t, pos_offset=0, out=None, out_f32=None):
    rows = x.shape[0]
    if out is None:
        od = x.dtype if out_f32 is None else (F32 if out_f32 else BF16)
        out = torch.empty(rows, x.shape[1], dtype=od, device=x.device)
    _lib.call("svla_rope", _ptr(x), _ld(x), _ptr(out), _ld(out), rows, heads, _ptr(cos_t),
              _ptr(sin_t), int(pos_offset), int(x.dtype == F32), int(out.dtype == F32), _stream())
    return out


def rope_table(max_pos, head_dim, theta, device=None):
    dev = device or torch.device("cuda")
    c = torch.empty(max_pos, head_dim // 2, dtype=F32, device=dev)
    s = torch.empty_like(c)
    _lib.call("svla_rope_table", _ptr(c), _ptr(s), max_pos, head_dim, float(theta), _stream())
    return c, s


def pack_weight(w_kn, out=None):
    """Reference ``[in, out]`` weight -> packed ``[out, in]`` on the device."""
    K, N = w_kn.shape
    out = torch.empty(N, K, dtype=BF16, device=w_kn.device) if out is None else out
    _lib.call("svla_pack_weight_bf16", _ptr(w_kn), _ld(w_kn), _ptr(out), K, N, _stream())
    return out


def pack_gate_up(w_gate, w_up, out=None):
    K, inter = w_gate.shape
    out = torch.empty(2 * inter, K, dtype=BF16, device=w_gate.device) if out is None else out
    _lib.call("svla_pack_gate_up_bf16", _ptr(w_gate.contiguous()), _ptr(w_up.contiguous()),
              _ptr(out), K, inter, _stream())
    return out


def embed(ids, table, scale, out, per_sample=None, out_bs=0):
    """Rows ``r`` of ``ids`` (flattened int64) -> ``out`` (2-D view with
    leading dim), sample ``r // per_sample`` offset by ``out_bs`` elements."""
    ids = ids.reshape(-1).to(torch.int64)
    n = ids.numel()
    per = n if per_sample is None else per_sample
    _lib.call("svla_embed_bf16", _ptr(ids), _ptr(table), table.shape[0], table.shape[1],
              float(scale), _ptr(out),
              _ld(out), int(out_bs), n, per, _stream())
    return out


def time_embedding(t, dim, out=None, min_period=4e-3, max_period=4.0, device=None):
    out = torch.empty(dim, dtype=BF16, device=device or "cuda") if out is None else out
    _lib.call("svla_time_embedding_bf16", float(t), dim, float(min_period), float(max_period),
              _ptr(out), _stream())
    return out


def f32_to_bf16(x, out=None):
    out = torch.empty(x.shape, dtype=BF16, device=x.device) if out is None else out
    _lib.call("svla_f32_to_bf16", _ptr(x), _ptr(out), x.numel(), _stream())
    return out


def image_to_bf16(frames, out_size=512, out=None):
    """uint8 RGB frames ``[n, h, w, 3]`` (GPU) -> bf16 ``[n, 3, S, S]`` in
    [-1, 1], aspect-preserving bilinear resize with black padding
    (``svla_image_to_bf16``)."""
    if frames.dtype != torch.uint8 or frames.dim() != 4 or frames.shape[-1] != 3:
        raise ValueError("frames must be uint8 [n, h, w, 3]")
    frames = frames.contiguous()
    n, h, w, _ = frames.shape
    if out is None:
        out = torch.empty(n, 3, out_size, out_size, dtype=BF16, device=frames.device)
    _lib.call("svla_image_to_bf16", _ptr(frames), h * w * 3, n, h, w, _ptr(out), out_size,
              _stream())
    return out


# ------------------------------------------------------ harness variants ---
UNARY = {"silu": 0, "gelu_tanh": 1, "gelu_erf": 2, "sin": 3, "cos": 4}
NORM_KIND = {"rms": 0, "rms_add": 1, "layer": 2}


def unary(x, op, out=None):
    """Elementwise ``op`` (silu, gelu_tanh, gelu_erf, sin, cos) on a contiguous
    fp32 or bf16 tensor, computed in fp32, same dtype out."""
    if x.dtype not in (F32, BF16) or not x.is_contiguous():
        raise ValueError("unary: contiguous fp32 or bf16 tensor expected")
    out = torch.empty_like(x) if out is None else out
    if out.dtype != x.dtype or not out.is_contiguous() or out.numel() != x.numel():
        raise ValueError("unary: out must match x")
    name = "svla_unary_f32" if x.dtype == F32 else "svla_unary_bf16"
    _lib.call(name, _ptr(x), _ptr(out), x.numel(), UNARY[op], _stream())
    return out


def add(x, y, out=None):
    """bf16 elementwise x + y (contiguous, same shape)."""
    if x.dtype != BF16 or y.dtype != BF16 or x.shape != y.shape:
        raise ValueError("add: two bf16 tensors of one shape expected")
    x, y = x.contiguous(), y.contiguous()
    out = torch.empty_like(x) if out is None else out
    _lib.call("svla_add_bf16", _ptr(x), _ptr(y), _ptr(out), x.numel(), _stream())
    return out


def row_norm(x, w, eps, kind, b=None, round_ops=False, out=None):
    """Row norm (kind rms / rms_add / layer) of a 2-D fp32 or bf16 tensor, all
    operands of x's dtype."""
    rows, cols = x.shape
    out = torch.empty_like(x) if out is None else out
    for t in (w, b, out):
        if t is not None and t.dtype != x.dtype:
            raise ValueError("row_norm: operands must share x's dtype")
    _lib.call("svla_row_norm", _ptr(x), _ld(x), _ptr(w), _ptr(b), _ptr(out), _ld(out), rows,
              cols, float(eps), NORM_KIND[kind], int(x.dtype == F32), int(round_ops), _stream())
    return out


def softmax_rows(s, row_start=-1, row_div=1, out=None, out_f32=None):
    """Row softmax of a 2-D fp32 / bf16 view with the causal limit
    ``c <= row_start + r // row_div`` (row_start < 0: unmasked)."""
    rows, cols = s.shape
    if out is None:
        dt = (F32 if out_f32 else BF16) if out_f32 is not None else s.dtype
        out = torch.empty(rows, cols, dtype=dt, device=s.device)
    _lib.call("svla_softmax_rows", _ptr(s), _ld(s), _ptr(out), _ld(out), rows, cols,
              int(row_start), int(row_div), int(s.dtype == F32), int(out.dtype == F32), _stream())
    return out


def conv_patch_f32(images, kernel, bias=None, out=None):
    """fp32 Conv2d(k = stride = patch): images [n, C, H, W], kernel [E, C, P, P]
    -> [n * (H/P) * (W/P), E]."""
    n, c, h, w = images.shape
    e, c2, pk, pk2 = kernel.shape
    if c2 != c or pk != pk2 or images.dtype != F32 or kernel.dtype != F32:
        raise ValueError("conv_patch_f32: fp32 images [n,C,H,W] and kernel [E,C,P,P] expected")
    images, kernel = images.contiguous(), kernel.contiguous()
    out = (torch.empty(n * (h // pk) * (w // pk), e, dtype=F32, device=images.device)
           if out is None else out)
    _lib.call("svla_conv_patch_f32", _ptr(images), _ptr(kernel), _ptr(bias), _ptr(out), n, c, h,
              w, pk, e, _stream())
    return out
