"""Per-kernel census of one chunk: every ``libsvla`` call of an eager chunk
with its algorithmic work (FLOPs for the MFMA contractions, HBM bytes for the
rest), timed per launch, grouped by kernel and shape.

How a call is timed: the calls of one group (same entry point, shape and
epilogue) are replayed in chunk order inside one captured HIP graph -- so
Python launch overhead never sits between them, and consecutive launches
touch different layers' weights as they do in a chunk -- and the graph's
replay time is divided by the number of launches.

Short groups are repeated inside their graph (16 launches at least), so the
graph's own launch cost does not land on a single kernel.

Work model (the units of the roofline fractions): a GEMM is 2 M N K FLOPs
and reads A and W once and writes C once (+ residual / bias / norm gains);
attention is 4 Sq Sk head_dim FLOPs per (sample, head), causal or not (dense
count, as the chunk's FLOP total); norms, casts and elementwise kernels are
their bytes read + written; the fused expert is the FLOPs of its Euler steps
and the weights it streams once per step.
"""

from __future__ import annotations

import ctypes
import statistics
from dataclasses import dataclass, field

import torch

from . import _lib

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
N_SIMD = 256 * 4            # MI355X: 256 CUs x 4 SIMDs
N_XCD = 8                   # GRBM_GUI_ACTIVE reads the sum over the 8 XCDs
# FETCH_SIZE (KiB) reads half the bytes a plain 1 GiB device copy moves on the
# MI355X boxes measured (calibration committed with the dominant kernel's
# traffic record): bytes = FETCH_SIZE x 1024 x FETCH_SCALE
FETCH_SCALE = 2.0


def _v(a):
    """Python value of a recorded ctypes argument."""
    return a.value if isinstance(a, (ctypes.c_void_p, ctypes.c_int, ctypes.c_long,
                                     ctypes.c_float, ctypes.c_double)) else a


def expert_step_flops(cfg, batch):
    """FLOPs of one Euler step of the action expert (dense attention count)."""
    d, e = cfg.decoder, cfg.expert
    A, L = cfg.chunk, cfg.prefix_len
    n_cross = sum(cfg.is_cross(i) for i in range(cfg.expert_layers))
    common = 2 * A * e.hidden * e.q_dim + 3 * 2 * A * e.inter * e.hidden
    self_l = common + 2 * A * 2 * e.kv_dim * e.hidden + 4 * A * A * e.n_q_heads * 64
    cross_l = common + 4 * A * L * e.n_q_heads * 64
    io = 2 * A * e.hidden * (cfg.action_dim + 2 * e.hidden) + 2 * A * cfg.action_dim * e.hidden
    return batch * ((cfg.expert_layers - n_cross) * self_l + n_cross * cross_l + io)


def expert_step_weight_bytes(cfg):
    """bf16 weight bytes one Euler step streams (every projection once)."""
    e = cfg.expert
    H = e.hidden
    total = 0
    for i in range(cfg.expert_layers):
        qkv = e.q_dim if cfg.is_cross(i) else e.q_dim + 2 * e.kv_dim
        total += (qkv * H + e.q_dim * H + 2 * e.inter * H + e.inter * H) * 2
    return total + (cfg.action_dim * H + 2 * H * H + H * cfg.action_dim) * 2


def work(name, args, cfg, batch):
    """(bound, flops, bytes, label) of one recorded call."""
    a = [_v(x) for x in args]
    if name in ("svla_linear_bf16", "svla_linear_scratch_bf16", "svla_linear_wide_bf16"):
        m, n, k = a[10], a[11], a[12]
        res, bias, out_f32 = a[6], a[4] or a[5], (a[15] if name != "svla_linear_wide_bf16" else 0)
        norm = a[16] if name != "svla_linear_wide_bf16" else None
        act = a[14]
        by = 2 * (m * k + n * k) + (4 if out_f32 else 2) * m * n + (2 * m * n if res else 0)
        by += (2 * k if norm else 0) + (2 * n if bias else 0)
        tag = "".join([" norm" if norm else "", " bias" if bias else "", f" act{act}" if act else "",
                       " +res" if res else "", " f32out" if out_f32 else ""])
        kind = "linear_wide" if name == "svla_linear_wide_bf16" else "linear"
        return "mfma", 2 * m * n * k, by, f"{kind} {m}x{n}x{k}{tag}"
    if name in ("svla_linear_rope_bf16", "svla_linear_rope_lo_bf16"):
        lo = name == "svla_linear_rope_lo_bf16"
        m, n, k = (a[7], a[8], a[9]) if lo else (a[6], a[7], a[8])
        norm, rc = (a[14], a[10]) if lo else (a[13], a[9])
        has_lo = lo and bool(a[5])
        by = 2 * (m * k + n * k + m * n) + (2 * k if norm else 0) + (2 * m * rc if has_lo else 0)
        return ("mfma", 2 * m * n * k, by,
                f"linear+rope {m}x{n}x{k}{' norm' if norm else ''}{' +lo' if has_lo else ''}")
    if name == "svla_linear_silu_mul_bf16":
        m, inter, k = a[6], a[7], a[8]
        by = 2 * (m * k + 2 * inter * k + m * inter) + (2 * k if a[9] else 0)
        return ("mfma", 2 * m * 2 * inter * k, by,
                f"linear gate|up+silu*mul {m}x{2 * inter}x{k}{' norm' if a[9] else ''}")
    if name == "svla_patch_embed_bf16":
        n_img, ch, img, p, emb = a[6], a[7], a[8], a[9], a[10]
        t = (img // p) ** 2
        kk = ch * p * p
        by = 2 * (n_img * ch * img * img + emb * kk + 2 * n_img * t * emb)
        return "mfma", 2 * n_img * t * emb * kk, by, f"patch embed {n_img * t}x{emb}x{kk}"
    if name == "svla_connector_bf16":
        n_img, grid, hid, sc, n_out = a[5], a[6], a[7], a[8], a[9]
        m, kk = n_img * (grid // sc) ** 2, hid * sc * sc
        by = 2 * (n_img * grid * grid * hid + n_out * kk + m * n_out)
        return "mfma", 2 * m * n_out * kk, by, f"connector {m}x{n_out}x{kk}"
    if name == "svla_action_out_euler":
        m, n, k = a[8], a[9], a[10]
        by = 2 * (m * k + n * k) + 10 * m * n
        return "mfma", 2 * m * n * k, by, f"action out+euler {m}x{n}x{k}"
    if name in ("svla_attention_bf16", "svla_attention_lo_bf16"):
        if name == "svla_attention_lo_bf16":
            b, sq, sk, hq, hkv, hd, mask = a[14], a[15], a[16], a[17], a[18], a[19], a[21]
            nlo = bool(a[1]) + bool(a[5])
        else:
            b, sq, sk, hq, hkv, hd, mask = a[12], a[13], a[14], a[15], a[16], a[17], a[19]
            nlo = 0
        by = 2 * b * (2 * sq * hq * hd + 2 * sk * hkv * hd)
        by += 2 * b * ((sq * hq * hd if nlo >= 1 else 0) + (sk * hkv * hd if nlo == 2 else 0))
        what = {0: "full", 1: "causal", 2: "prefix"}.get(mask, f"mask{mask}")
        return ("mfma", 4 * b * hq * sq * sk * hd, by,
                f"attention b{b} {sq}x{sk} {hq}/{hkv} heads {what}{' +lo' * nlo}")
    if name == "svla_expert_run":
        steps = cfg.num_steps
        by = steps * expert_step_weight_bytes(cfg)
        return ("hbm", steps * expert_step_flops(cfg, batch), by,
                f"fused action expert ({steps} Euler steps, batch {batch})")
    if name == "svla_rmsnorm_bf16":
        r, c = a[5], a[6]
        return "hbm", 0, 2 * (2 * r * c + c), f"rmsnorm {r}x{c}"
    if name == "svla_layernorm_bf16":
        r, c = a[6], a[7]
        return "hbm", 0, 2 * (2 * r * c + 2 * c), f"layernorm {r}x{c}"
    if name == "svla_layernorm_blocked_bf16":
        r, c = a[5], a[6]
        return "hbm", 0, 2 * (2 * r * c + 2 * c), f"layernorm->blocked {r}x{c}"
    if name == "svla_slab_block_bf16":
        r, k = a[3], a[4]
        return "hbm", 0, 4 * r * k, f"slab block {r}x{k}"
    if name == "svla_embed_bf16":
        hid, n_tok = a[3], a[8]
        return "hbm", 0, 4 * n_tok * hid, f"token embed {n_tok}x{hid}"
    if name == "svla_image_to_bf16":
        n, h, w, out = a[2], a[3], a[4], a[6]
        return "hbm", 0, n * h * w * 3 + 2 * n * 3 * out * out, f"image -> bf16 {n}x{h}x{w}"
    if name == "svla_add_bf16":
        return "hbm", 0, 6 * a[3], f"add {a[3]}"
    if name in ("svla_silu_bf16", "svla_f32_to_bf16"):
        return "hbm", 0, 4 * a[2], f"{name[5:]} {a[2]}"
    if name == "svla_silu_mul_bf16":
        return "hbm", 0, 6 * a[3], f"silu*mul {a[3]}"
    if name == "svla_gelu_bf16":
        return "hbm", 0, 4 * a[2], f"gelu {a[2]}"
    return "hbm", 0, 0, name[5:]


@dataclass
class Group:
    label: str
    name: str
    bound: str
    flops: float
    bytes: float
    calls: list = field(default_factory=list)
    us: float = 0.0          # per launch

    @property
    def n(self):
        return len(self.calls)

    def row(self):
        per_s = self.us * 1e-6
        if self.bound == "mfma":
            ach = self.flops / per_s / 1e12
            return ach, ach / PEAK_BF16_TFLOPS, "TFLOP/s"
        ach = self.bytes / per_s / 1e9
        return ach, ach / PEAK_HBM_GBS, "GB/s"


# entry points that set state rather than launch work: not timed
_SKIP = {"svla_init", "svla_version", "svla_gemm_set_tile", "svla_gemm_set_split",
         "svla_gemm_tile_choice", "svla_expert_workspace_size", "svla_expert_prepare",
         "svla_expert_status", "svla_time_embedding_bf16", "svla_rope_table"}


def record_chunk(eng):
    """The libsvla calls of one eager chunk of ``eng`` (a SmolVLAEngine with
    ``use_graph=False``), in order."""
    calls = []

    def hook(name, args, run):
        if name not in _SKIP:
            calls.append((name, args))
        return run()

    _lib.set_observer(hook)
    try:
        eng.step()
        torch.cuda.synchronize()
    finally:
        _lib.set_observer(None)
    return calls


def _launch(name, args):
    """Launch a recorded call on the current stream."""
    argv = list(args)
    argv[-1] = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = getattr(_lib.load(), name)(*argv)
    if rc != 0:
        raise _lib.SvlaError(f"{name}: replay failed ({rc})")


def group_calls(calls, cfg, batch):
    groups = {}
    for name, args in calls:
        bound, fl, by, label = work(name, args, cfg, batch)
        g = groups.get(label)
        if g is None:
            g = groups[label] = Group(label, name, bound, fl, by)
        g.calls.append(args)
    return list(groups.values())


def time_groups(groups, reps=3):
    """Per-launch time of every group (HIP-graph replay of its calls)."""
    for g in groups:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for args in g.calls:        # warm-up, eager
                _launch(g.name, args)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        # short groups repeat inside the graph: a graph launch costs ~20 us,
        # which must not land on a single kernel
        rounds = max(1, -(-16 // g.n))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(rounds):
                for args in g.calls:
                    _launch(g.name, args)
        graph.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            graph.replay()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b))
        g.us = statistics.median(ts) * 1e3 / (g.n * rounds)
        del graph
    return groups


def table(groups, top=25):
    """Markdown rows of the ``top`` groups by time per chunk."""
    total = sum(g.us * g.n for g in groups)
    rows = ["| # | kernel (entry point: shape, epilogue) | launches | us / launch | "
            "ms / chunk | % | work / launch | achieved | peak fraction |",
            "|---:|---|---:|---:|---:|---:|---:|---:|---:|"]
    for i, g in enumerate(sorted(groups, key=lambda g: -g.us * g.n)[:top], 1):
        ach, frac, unit = g.row()
        wk = (f"{g.flops / 1e9:.3f} GFLOP" if g.bound == "mfma" else f"{g.bytes / 1e6:.3f} MB")
        rows.append(f"| {i} | `{g.name}`: {g.label} | {g.n} | {g.us:.2f} | {g.us * g.n / 1e3:.3f} | "
                    f"{100 * g.us * g.n / total:.1f} | {wk} | {ach:.1f} {unit} | "
                    f"{frac:.3f} ({'MFMA' if g.bound == 'mfma' else 'HBM'}) |")
    return "\n".join(rows), total / 1e3


# ------------------------------------------------------------------------------
# In-chunk profile: the kernels of one graph-replayed chunk, as a profiler sees
# them, matched to the libsvla calls of the chunk (same order), so every census
# group gets its in-chunk time and hardware counters beside its isolated replay.

# kernel-name prefixes a call may dispatch, in order (one kernel per call
# unless listed otherwise)
_FAMILIES = {
    "svla_linear_wide_bf16": [("gemm_wide_kernel",)],
    "svla_attention_bf16": [("attention_",)],
    "svla_attention_lo_bf16": [("attention_",)],
    "svla_expert_run": [("clear_u32_kernel",), ("expert_kernel",)],
    "svla_rmsnorm_bf16": [("rmsnorm_kernel",)],
    "svla_layernorm_bf16": [("layernorm_kernel",)],
    "svla_layernorm_blocked_bf16": [("layernorm_kernel",)],
}
_GEMM = ("gemm_", "skinny_kernel")


def dispatch_families(name):
    """Kernel-name prefixes of the dispatches one call makes, in order."""
    if name in _FAMILIES:
        return _FAMILIES[name]
    if name.startswith(("svla_linear", "svla_patch", "svla_connector", "svla_action_out")):
        return [_GEMM]
    return [("",)]  # any one kernel


def call_list(calls, cfg, batch):
    """[(entry point, bound, flops, bytes, group label)] of recorded calls."""
    return [(name, *work(name, args, cfg, batch)) for name, args in calls]


def short_kernel_name(n):
    """``void (anonymous namespace)::gemm_line_kernel<...>(GemmArgs)`` ->
    ``gemm_line_kernel<...>``."""
    import re
    n = n.replace("void ", "").replace("(anonymous namespace)::", "")
    return re.sub(r"\((?:[^()]|\([^()]*\))*\)$", "", n).strip()


def own_dispatches(rows):
    """Profiler rows of this library's kernels, in dispatch order: they live
    in top-level anonymous namespaces (torch's kernels sit in named ones, the
    runtime's copies in none)."""
    return [r for r in rows
            if r["Kernel_Name"].replace("void ", "", 1).startswith("(anonymous namespace)::")]


def align_last_chunk(calls, dispatches):
    """Match the last len(expanded calls) library dispatches to the calls:
    returns [(call index, dispatch row)]; raises if a kernel family does not
    match its call."""
    fam = [(i, f) for i, c in enumerate(calls) for f in dispatch_families(c[0])]
    if len(dispatches) < len(fam):
        raise ValueError(f"{len(dispatches)} dispatches for {len(fam)} expected")
    tail = dispatches[len(dispatches) - len(fam):]
    out = []
    for (i, f), r in zip(fam, tail):
        k = short_kernel_name(r["Kernel_Name"])
        if not k.startswith(f):
            raise ValueError(f"call {i} ({calls[i][0]}) expects {f}, profiler shows {k}")
        out.append((i, r))
    return out


def profile_table(calls, iso_us, trace_rows, pmc_rows, batch):
    """Markdown of the in-chunk profile: per census group, the isolated replay
    time, the in-chunk time (last replayed chunk of the kernel trace) and the
    counter-derived figures (per dispatch, averaged over the group's launches
    in the last eager chunk of each counter run)."""
    import collections
    al = align_last_chunk(calls, own_dispatches(trace_rows))
    dur = collections.defaultdict(float)
    kern, kern_us = {}, {}
    for i, r in al:
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        dur[i] += us
        # a call with several dispatches (the fused expert's clear + launch)
        # is labelled by its longest one
        if us > kern_us.get(calls[i][4], -1.0):
            kern[calls[i][4]], kern_us[calls[i][4]] = short_kernel_name(r["Kernel_Name"]), us
    # counters: {call index: {counter: value}} from every counter run
    cnt = collections.defaultdict(dict)
    for rows in pmc_rows:
        per = collections.OrderedDict()
        for r in rows:
            key = int(r["Dispatch_Id"])
            d = per.setdefault(key, {"Kernel_Name": r["Kernel_Name"], "c": {}})
            d["c"][r["Counter_Name"]] = d["c"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        disp = [{"Kernel_Name": v["Kernel_Name"], "c": v["c"]} for _, v in sorted(per.items())]
        for i, d in align_last_chunk(calls, own_dispatches(disp)):
            for k, v in d["c"].items():     # a call's dispatches add up
                cnt[i][k] = cnt[i].get(k, 0.0) + v
    groups = collections.OrderedDict()
    for i, (name, bound, fl, by, label) in enumerate(calls):
        g = groups.setdefault(label, {"name": name, "bound": bound, "flops": fl, "bytes": by,
                                      "idx": []})
        g["idx"].append(i)
    total = sum(dur.values())

    def avg(g, key):
        vals = [cnt[i][key] for i in g["idx"] if key in cnt[i]]
        return sum(vals) / len(vals) if vals else None

    rows = ["| # | group (entry point: shape, epilogue) | kernel | launches | isolated us | "
            "in-chunk us | ms / chunk | % | in-chunk peak fraction | MFMA busy | issuing | "
            "waiting | L2 hit | fetched / algorithmic |",
            "|---:|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    order = sorted(groups.items(), key=lambda kv: -sum(dur[i] for i in kv[1]["idx"]))
    ratio = lambda a, b, k=1.0: f"{k * a / b:.2f}" if a is not None and b else "-"  # noqa: E731
    for n, (label, g) in enumerate(order[:30], 1):
        t = sum(dur[i] for i in g["idx"])
        us = t / len(g["idx"])
        if g["bound"] == "mfma":
            frac = g["flops"] / (us * 1e-6) / (PEAK_BF16_TFLOPS * 1e12)
        else:
            frac = g["bytes"] / (us * 1e-6) / (PEAK_HBM_GBS * 1e9)
        wc = avg(g, "SQ_WAVE_CYCLES")
        hit, miss = avg(g, "TCC_HIT"), avg(g, "TCC_MISS")
        gui = avg(g, "GRBM_GUI_ACTIVE")
        iso = iso_us.get(label)
        rows.append(
            f"| {n} | `{g['name']}`: {label} | `{kern.get(label, '?')[:56]}` | {len(g['idx'])} | "
            f"{f'{iso:.2f}' if iso is not None else '-'} | {us:.2f} | {t / 1e3:.3f} | "
            f"{100 * t / total:.1f} | {frac:.3f} ({'MFMA' if g['bound'] == 'mfma' else 'HBM'}) | "
            f"{ratio(avg(g, 'SQ_VALU_MFMA_BUSY_CYCLES'), gui / N_XCD * N_SIMD if gui else None)} | "
            f"{ratio(avg(g, 'SQ_ACTIVE_INST_ANY'), wc)} | {ratio(avg(g, 'SQ_WAIT_ANY'), wc)} | "
            f"{ratio(hit, (hit + miss) if hit is not None and miss is not None else None)} | "
            f"{ratio(avg(g, 'FETCH_SIZE'), g['bytes'], 1024 * FETCH_SCALE)} |")
    return "\n".join(rows), total / 1e3, len(al)
