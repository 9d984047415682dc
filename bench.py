"""SmolVLA bf16 inference benchmark on one MI355X.

Workload: BASELINE config 4 -- full SmolVLA inference (3 cameras at 512x512,
48 language tokens, 32-dim state -> SigLIP ViT x12 -> pixel-shuffle connector ->
16-layer prefix with KV cache -> 10 Euler steps of the 16-layer action expert
-> 50x32 action chunk), random-init bf16 weights, synthetic inputs already
resident in HBM.  A "step" is one chunk for the whole batch (one HIP-graph
replay).

Prints ONE JSON line:
  value        chunks/s at batch 32 (whole job; higher is better)
  latency      ms per chunk at batch 1 (median of >= 50 chunks)
  latency_bs1  ms per chunk at batch 1, with its roofline: the chunk's floor
               = max(FLOPs / MFMA peak, bytes / HBM peak) (every weight once,
               the expert's re-read per Euler step) against the median time
  roofline     the dominant kernel -- the (entry point, shape, epilogue) group
               with the most time per batch-32 chunk in a live census of one
               chunk (smolvla.census): algorithmic FLOPs (or bytes) / average
               launch time from HIP events on its stream, against the 2.5 PFLOP/s
               dense bf16 (or 8 TB/s HBM) peak
  cpu_baseline the CPU oracle (PyTorch bf16 restatement of the reference
               modules) timed on this host's cores on a bounded sample of
               bs=1 chunks (the bs=32 CPU rate extrapolated as bs=1 x 32)
  configs_bs1  BASELINE configs 0-3 at batch 1: GPU latency (HIP-graph
               replays), roofline floor and fraction, and the CPU oracle's
               time for the same config in the same run, with its threads
  output_check the timed engine's actions are finite and sample 0 matches the
               batch-1 engine (checked outside every timed region)
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (str(ROOT / "vla-to-npu_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# final actions, engine vs engine or vs the oracle (the chunk tests' bound)
OUTPUT_ATOL = 5e-2


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def chunk_flops(cfg, batch):
    """Algorithmic FLOPs of one chunk (2*M*N*K per GEMM, attention counted
    dense: 2 * 2 * Sq * Sk * heads * 64)."""
    v, d, e = cfg.vit, cfg.decoder, cfg.expert
    T, H = v.tokens, v.hidden
    vit = 2 * T * (3 * H) * H + 2 * T * H * H + 2 * 2 * T * v.inter * H + 4 * T * T * v.n_heads * 64
    patch = 2 * T * H * (v.channels * v.patch ** 2)
    img = cfg.n_cameras * (vit * v.layers + patch)
    conn = cfg.n_cameras * 2 * cfg.image_tokens * d.hidden * H * cfg.pixel_shuffle ** 2
    L = cfg.prefix_len
    dec = (2 * L * (d.q_dim + 2 * d.kv_dim) * d.hidden + 2 * L * d.hidden * d.q_dim
           + 3 * 2 * L * d.inter * d.hidden + 4 * L * L * d.n_q_heads * 64)
    prefix = cfg.prefix_layers * dec + 2 * d.hidden * cfg.state_dim
    n_cross = sum(cfg.is_cross(i) for i in range(cfg.expert_layers))
    cross_kv = n_cross * 2 * 2 * L * d.kv_dim * d.kv_dim
    A = cfg.chunk
    common = 2 * A * e.hidden * e.q_dim + 3 * 2 * A * e.inter * e.hidden
    self_l = common + 2 * A * 2 * e.kv_dim * e.hidden + 4 * A * A * e.n_q_heads * 64
    cross_l = common + 4 * A * L * e.n_q_heads * 64
    io = 2 * A * e.hidden * (cfg.action_dim + 2 * e.hidden) + 2 * A * cfg.action_dim * e.hidden
    step = (cfg.expert_layers - n_cross) * self_l + n_cross * cross_l + io
    return batch * (img + conn + prefix + cross_kv + cfg.num_steps * step)


def time_chunks(eng, n):
    """Per-chunk wall times (ms) from HIP events on the engine's stream."""
    out = []
    for _ in range(n):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        eng.step()
        b.record()
        b.synchronize()
        out.append(a.elapsed_time(b))
    return out


def _up_proj_launcher(cfg, M, x, w_packed, bias):
    """The ViT MLP up-projection exactly as the engine launches it at this
    row count (``layers.vit_blocked_plan``): on the 256x256 kernel with
    slab-blocked activations (the LayerNorm writes them so) and weights, and
    a slab-blocked output when the down-projection reads it so; else through
    ``ops.linear``."""
    from smolvla import layers, ops
    v = cfg.vit
    plan = layers.vit_blocked_plan(v.hidden, v.inter, M)
    if plan["up"]:
        xb = ops.slab_block(x)
        wb = ops.slab_block(w_packed)
        lay = ops.LAYOUT_A_BLOCKED | ops.LAYOUT_W_BLOCKED
        if plan["down"]:
            lay |= ops.LAYOUT_C_BLOCKED
            out = torch.empty(v.inter // 32, M, 32, device="cuda", dtype=torch.bfloat16)
        else:
            out = torch.empty(M, v.inter, device="cuda", dtype=torch.bfloat16)
        return lambda: ops.linear_wide(xb, wb, M, v.inter, v.hidden, bias=bias,
                                       act="gelu_" + v.gelu, out=out, layout=lay)
    out = torch.empty(M, v.inter, device="cuda", dtype=torch.bfloat16)
    return lambda: ops.linear(x, w_packed, bias=bias, act="gelu_" + v.gelu, out=out)


def census_groups(eng):
    """Group and time every libsvla call of one eager chunk of ``eng``."""
    from smolvla import census
    was = eng.use_graph
    eng.use_graph = False
    try:
        census.record_chunk(eng)           # warm-up
        calls = census.record_chunk(eng)
    finally:
        eng.use_graph = was
    groups = census.group_calls(calls, eng.cfg, eng.B)
    return census.time_groups(groups)


def dominant_roofline(eng):
    """Roofline line of the group with the most time per chunk."""
    from smolvla import census
    groups = census_groups(eng)
    top = max(groups, key=lambda g: g.us * g.n)
    ach, frac, unit = top.row()
    total_us = sum(g.us * g.n for g in groups)
    rec = {"kernel": f"{top.name}: {top.label}", "launches_per_chunk": top.n,
           "share_of_chunk": round(top.us * top.n / total_us, 4),
           "bound": top.bound, "achieved": round(ach, 1),
           "peak": PEAK_BF16_TFLOPS if top.bound == "mfma" else PEAK_HBM_GBS, "unit": unit,
           "frac": round(frac, 4), "avg_launch_us": round(top.us, 2),
           "algorithmic_flops": top.flops, "algorithmic_bytes": top.bytes, "traffic": None}
    tr = load_traffic()
    m = top.label.split()[1] if top.label.startswith(("linear", "linear_wide")) else None
    if tr and m and "x".join(map(str, tr.get("shape", []))) == m:
        rec["traffic"] = tr.get("bytes_per_launch")
    return rec, groups


TRAFFIC_FILE = ROOT / "profiles" / "dominant_kernel_traffic.json"


def traffic_probe(cfg, batch):
    """Counter-collection entry point (run under ``rocprofv3 --pmc FETCH_SIZE``
    and again under ``--pmc WRITE_SIZE``): the dominant kernel alone at its
    batch-``batch`` shape, 3 launches, then a plain 1 GiB device copy, 3
    launches, whose known byte count calibrates the counters."""
    from smolvla import ops
    v = cfg.vit
    M = batch * cfg.n_cameras * v.tokens
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(M, v.hidden, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(v.inter, v.hidden, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(v.inter, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    run = _up_proj_launcher(cfg, M, x, w, b)
    torch.cuda.synchronize()
    for _ in range(3):
        run()
    src = torch.ones(1 << 29, device="cuda", dtype=torch.bfloat16)   # 1 GiB
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"traffic probe done: GEMM {M}x{v.inter}x{v.hidden}, copy 1 GiB")


def load_traffic():
    """HBM bytes per launch of the dominant kernel, measured by the
    FETCH_SIZE / WRITE_SIZE counter runs of ``--traffic-probe`` (scaled by the
    copy calibration) and committed with their rocprofv3 summary; None when
    absent."""
    try:
        return json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None


def traffic_summary(fetch_csv, write_csv, shape):
    """Write the committed traffic record from the two ``--traffic-probe``
    counter runs' ``*_counter_collection.csv`` files: per dispatch of the GEMM
    and of the 1 GiB copy, FETCH_SIZE / WRITE_SIZE in KiB; each counter is
    scaled so that the copy reads (resp. writes) exactly 1 GiB."""
    import csv

    def per_dispatch(path, counter):
        vals = {}
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if r.get("Counter_Name") != counter:
                    continue
                name = r["Kernel_Name"]
                kind = "gemm" if "gemm" in name else "copy" if "copyBuffer" in name else None
                if kind:
                    key = (kind, r.get("Dispatch_Id") or r.get("Correlation_Id"))
                    vals[key] = (name, vals.get(key, (name, 0.0))[1] + float(r["Counter_Value"]))
        out = {"gemm": [], "copy": [], "name": None}
        for (kind, _), (name, v) in sorted(vals.items(), key=lambda kv: int(kv[0][1])):
            out[kind].append(v)
            if kind == "gemm":
                out["name"] = name
        return out

    fe, wr = per_dispatch(fetch_csv, "FETCH_SIZE"), per_dispatch(write_csv, "WRITE_SIZE")
    gib_kib = float(1 << 20)
    fscale = gib_kib / statistics.mean(fe["copy"])
    wscale = gib_kib / statistics.mean(wr["copy"])
    fb = statistics.mean(fe["gemm"]) * fscale * 1024
    wb = statistics.mean(wr["gemm"]) * wscale * 1024
    M, N, K = shape
    kname = fe["name"].replace("(anonymous namespace)::", "").replace("void ", "")
    rec = {"kernel": kname.split("(")[0].strip(), "shape": list(shape),
           "fetch_kib_raw": [round(v, 1) for v in fe["gemm"]],
           "write_kib_raw": [round(v, 1) for v in wr["gemm"]],
           "copy_fetch_kib_raw": [round(v, 1) for v in fe["copy"]],
           "copy_write_kib_raw": [round(v, 1) for v in wr["copy"]],
           "fetch_scale": round(fscale, 4), "write_scale": round(wscale, 4),
           "fetch_bytes": int(fb), "write_bytes": int(wb), "bytes_per_launch": int(fb + wb),
           "algorithmic_bytes": 2.0 * (M * K + N * K + M * N + N)}
    TRAFFIC_FILE.write_text(json.dumps(rec, indent=1) + "\n")
    print(json.dumps(rec))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def chunk_floor(cfg, params, batch=1):
    """(floor_us, bound, flops, bytes) of one chunk: max of FLOPs at the MFMA
    peak and bytes at the HBM peak, bytes = every weight once + the expert
    weights re-read by each later Euler step."""
    from smolvla import census
    flops = chunk_flops(cfg, batch)
    w = 0
    stack = [params]
    while stack:
        x = stack.pop()
        if isinstance(x, dict):
            stack.extend(x.values())
        elif isinstance(x, (list, tuple)):
            stack.extend(x)
        elif torch.is_tensor(x):
            w += x.numel() * x.element_size()
    by = w + (cfg.num_steps - 1) * census.expert_step_weight_bytes(cfg)
    t_mfma = flops / (PEAK_BF16_TFLOPS * 1e12) * 1e6
    t_hbm = by / (PEAK_HBM_GBS * 1e9) * 1e6
    return (max(t_mfma, t_hbm), "mfma" if t_mfma >= t_hbm else "hbm", flops, by)


def cpu_baseline(cfg, params, seconds):
    """CPU oracle (PyTorch bf16 restatement of the reference modules) on this
    host: bs=1 chunks until `seconds` of work (after one warm-up chunk)."""
    import oracle.smolvla_ref as ref
    from smolvla.params import smolvla_inputs
    torch.set_num_threads(min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "64"))))
    inputs = smolvla_inputs(cfg, 1, seed=7)
    with torch.inference_mode():
        ref.smolvla_chunk(*inputs, params, cfg)
        n, t0 = 0, time.perf_counter()
        while True:
            ref.smolvla_chunk(*inputs, params, cfg)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 50:
                break
    return {"value": round(n / el, 4), "unit": "chunks/s", "cores": torch.get_num_threads(),
            "kind": "port", "cpu_model": cpu_model(), "host_cpus": os.cpu_count(),
            "batch": 1, "extrapolated": "bs=1 x 32: the batch-32 CPU rate is taken as the "
                                        "measured bs=1 chunk rate (samples are independent)",
            "sample": f"{n} full bs=1 chunks (3x512^2 cameras, 241-token prefix, 10 Euler "
                      f"steps) in {el:.1f} s, torch {torch.__version__} bf16 on CPU; "
                      f"reported as the bs=32 rate by bs=1 x 32 extrapolation",
            "ms_per_chunk": round(el / n * 1e3, 1)}


def _tree_bytes(tree):
    """bf16 bytes of every tensor in a (nested) params tree."""
    n, stack = 0, [tree]
    while stack:
        x = stack.pop()
        if isinstance(x, dict):
            stack.extend(x.values())
        elif isinstance(x, (list, tuple)):
            stack.extend(x)
        elif torch.is_tensor(x):
            n += 2 * x.numel()
    return n


def graph_ms(fn, reps=50, warm=3):
    """(median, min) ms of ``reps`` HIP-graph replays of ``fn``'s launches."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warm):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b))
    del g
    return statistics.median(ts), min(ts)


def config_work(cfg, params):
    """(flops, bytes) of BASELINE configs 0-3 at batch 1: FLOPs as in
    ``chunk_flops`` (attention dense); bytes = every weight the config reads
    once plus its inputs and outputs."""
    from smolvla import census
    v, d, e = cfg.vit, cfg.decoder, cfg.expert
    T, H = v.tokens, v.hidden

    def dec_flops(L, dc):
        return (2 * L * (dc.q_dim + 2 * dc.kv_dim) * dc.hidden + 2 * L * dc.hidden * dc.q_dim
                + 3 * 2 * L * dc.inter * dc.hidden + 4 * L * L * dc.n_q_heads * 64)

    L0, Lp = 128, cfg.prefix_len
    vit = (2 * T * (3 * H) * H + 2 * T * H * H + 2 * 2 * T * v.inter * H
           + 4 * T * T * v.n_heads * 64)
    patch = 2 * T * H * (v.channels * v.patch ** 2)
    conn = cfg.n_cameras * 2 * cfg.image_tokens * d.hidden * H * cfg.pixel_shuffle ** 2
    kv_bytes = 2 * Lp * 2 * d.kv_dim
    n_cross = sum(cfg.is_cross(i) for i in range(cfg.expert_layers))
    step_b = census.expert_step_weight_bytes(cfg) + n_cross * 2 * Lp * 2 * e.kv_dim
    return {
        "cfg0": (dec_flops(L0, d), _tree_bytes(params["prefix"][0]) + 2 * L0 * (2 * d.hidden + 2 * d.kv_dim)),
        "cfg1": (v.layers * vit + patch, _tree_bytes([params["vit"], params["patch"]])
                 + 2 * (v.channels * v.image ** 2 + T * H)),
        "cfg2": (conn + cfg.prefix_layers * dec_flops(Lp, d) + 2 * d.hidden * cfg.state_dim,
                 _tree_bytes([params["connector"], params["prefix"], params["state"]])
                 + 2 * (cfg.n_cameras * T * H + cfg.lang_tokens * d.hidden)
                 + cfg.prefix_layers * kv_bytes),
        "cfg3_step": (census.expert_step_flops(cfg, 1), step_b),
        "cfg3_loop": (cfg.num_steps * census.expert_step_flops(cfg, 1), cfg.num_steps * step_b),
    }


CONFIG_NAMES = {
    "cfg0": "config 0: one SmolLM2 decoder block, 128 tokens, causal, KV out",
    "cfg1": "config 1: SigLIP ViT per image (patch embed + 12 blocks, 1024 tokens)",
    "cfg2": "config 2: connector x3 cameras + 241-token prefix x16 layers with KV cache",
    "cfg3_step": "config 3: one Euler step of the 16-layer action expert (layer by layer)",
    "cfg3_loop": "config 3: the 10-step expert loop (the fused batch-1 launch)",
}


def gpu_configs(cfg, params, e1):
    """BASELINE configs 0-3 at batch 1 on the GPU, on the prepared weights of
    the batch-1 engine ``e1``: each config's launches captured in one HIP
    graph, median of 50 replays."""
    from smolvla import layers, ops
    v, d = cfg.vit, cfg.decoder
    dev = e1.device
    g = torch.Generator(device=dev).manual_seed(11)
    # cfg0: the prefix's layer-0 weights at 128 tokens, causal
    x0 = torch.randn(128, d.hidden, generator=g, device=dev).to(torch.bfloat16)
    x = torch.empty_like(x0)
    kv = torch.empty(128, d.q_dim + 2 * d.kv_dim, dtype=torch.bfloat16, device=dev)
    rope128 = layers.Rope.make(128, d.head_dim, d.rope_theta, dev)
    bufs0 = layers.Buffers(dev)

    def cfg0():
        x.copy_(x0)
        layers.decoder_layer(x, e1.prefix[0], d, 1, 128, rope128, "causal", 0, bufs0, qkv_out=kv)

    img = e1.in_images[:1]
    vx = torch.empty(v.tokens, v.hidden, dtype=torch.bfloat16, device=dev)
    bufs1 = layers.Buffers(dev)

    def cfg1():
        ops.patch_embed(img, e1.patch_w, e1.patch_b, e1.pos_emb, v.patch, out=vx)
        for P in e1.vit:
            layers.vit_layer(vx, P, v, 1, v.tokens, bufs1)

    def cfg2():
        e1.build_prefix()
        e1.run_prefix()

    dt = -1.0 / cfg.num_steps

    def cfg3_step():
        e1.expert_step(0, dt)

    def cfg3_loop():
        e1.x_t.copy_(e1.in_noise.view(-1, cfg.action_dim))
        e1.fx.run()

    out = {}
    for name, fn in (("cfg0", cfg0), ("cfg1", cfg1), ("cfg2", cfg2), ("cfg3_step", cfg3_step),
                     ("cfg3_loop", cfg3_loop)):
        if name == "cfg3_loop" and e1.fx is None:
            continue
        med, mn = graph_ms(fn)
        out[name] = (med, mn)
        log(f"{name}: {med:.3f} ms (GPU, batch 1)")
    e1.check()
    return out


def cpu_configs(cfg, params, seconds=3.0):
    """The CPU oracle on BASELINE configs 0-3 at batch 1 (bf16, this host's
    cores): median of repeats until ``seconds`` per config (at least 3)."""
    import oracle.smolvla_ref as ref
    from smolvla.params import smolvla_inputs
    torch.set_num_threads(min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "64"))))
    g = torch.Generator().manual_seed(11)
    d, v = cfg.decoder, cfg.vit
    x0 = torch.randn(1, 128, d.hidden, generator=g).to(torch.bfloat16)
    images, ids, state, noise = smolvla_inputs(cfg, 1, seed=7)
    vis = torch.randn(1, cfg.n_cameras, v.tokens, v.hidden, generator=g).to(torch.bfloat16)
    with torch.inference_mode():
        prefix = ref.build_prefix(vis, ids, state, params, cfg)
        _, kvc = ref.prefix_forward(prefix, params, cfg)
        ckv = ref.cross_kv(kvc, params, cfg)

    def vit1():
        y = ref.patch_embed(images[0, :1], params["patch"]["kernel"], params["patch"]["bias"],
                            params["patch"]["pos_emb"])
        for lp in params["vit"]:
            y = ref.vit_block(y, lp, v)
        return y

    def pre():
        p = ref.build_prefix(vis, ids, state, params, cfg)
        return ref.prefix_forward(p, params, cfg)

    def loop():
        x, t = noise.clone(), 1.0
        for _ in range(cfg.num_steps):
            x = x + (-1.0 / cfg.num_steps) * ref.expert_velocity(x, t, ckv, params, cfg).float()
            t -= 1.0 / cfg.num_steps
        return x

    fns = {"cfg0": lambda: ref.decoder_block(x0, params["prefix"][0], d, "causal"),
           "cfg1": vit1, "cfg2": pre,
           "cfg3_step": lambda: ref.expert_velocity(noise, 1.0, ckv, params, cfg),
           "cfg3_loop": loop}
    out = {}
    with torch.inference_mode():
        for name, fn in fns.items():
            fn()                                   # warm-up
            ts, t_end = [], time.perf_counter() + seconds
            while len(ts) < 3 or (time.perf_counter() < t_end and len(ts) < 20):
                t0 = time.perf_counter()
                fn()
                ts.append((time.perf_counter() - t0) * 1e3)
            out[name] = (statistics.median(ts), len(ts))
            log(f"{name}: {out[name][0]:.1f} ms (CPU oracle, {torch.get_num_threads()} threads)")
    return out, torch.get_num_threads()


def config_lines(cfg, params, gpu, cpu, threads):
    work = config_work(cfg, params)
    lines = {}
    for name, (med, mn) in gpu.items():
        fl, by = work[name]
        t_mfma = fl / (PEAK_BF16_TFLOPS * 1e12) * 1e6
        t_hbm = by / (PEAK_HBM_GBS * 1e9) * 1e6
        floor = max(t_mfma, t_hbm)
        row = {"what": CONFIG_NAMES[name], "batch": 1, "gpu_ms_median": round(med, 4),
               "gpu_ms_min": round(mn, 4), "flops": fl, "bytes": by,
               "tflops": round(fl / (med * 1e-3) / 1e12, 2),
               "gbs": round(by / (med * 1e-3) / 1e9, 1),
               "roofline": {"bound": "mfma" if t_mfma >= t_hbm else "hbm",
                            "floor_us": round(floor, 2), "frac": round(floor / (med * 1e3), 4)}}
        if cpu and name in cpu:
            row["cpu_ms_median"] = round(cpu[name][0], 2)
            row["cpu_reps"] = cpu[name][1]
            row["cpu_threads"] = threads
            row["gpu_speedup_vs_cpu"] = round(cpu[name][0] / med, 1)
        lines[name] = row
    return lines


def write_kernel_table(cfg, params, batch):
    """profiles/kernel_table_bs<batch>.md: the census table of one chunk."""
    from smolvla import census
    from smolvla.params import smolvla_inputs
    from smolvla.pipeline import SmolVLAEngine
    eng = SmolVLAEngine(cfg, params, batch=batch)
    eng.load_inputs(*smolvla_inputs(cfg, batch, seed=1, device="cuda"))
    eng.capture()
    for _ in range(3):
        eng.step()
    ts = time_chunks(eng, 10)
    groups = census_groups(eng)
    rows, total_ms = census.table(groups)
    n_launch = sum(g.n for g in groups)
    path = ROOT / "profiles" / f"kernel_table_bs{batch}.md"
    path.write_text(
        f"# Per-kernel census: one SmolVLA chunk at batch {batch}\n\n"
        f"Command (repo root on the MI355X box): `python bench.py --kernel-table {batch}`\n\n"
        f"Every libsvla call of one eager chunk, grouped by entry point, shape and epilogue; a group's "
        f"calls are replayed in chunk order inside one HIP graph and timed with HIP events "
        f"(median of 3 replays / launches).  Work per launch as `smolvla/census.py` states it "
        f"(GEMM 2MNK FLOPs, attention 4 Sq Sk d per head, dense; bandwidth kernels bytes read + "
        f"written; the fused expert its Euler steps' FLOPs and streamed weights); fraction of the "
        f"2.5 PFLOP/s bf16 MFMA or 8 TB/s HBM peak.\n\n"
        f"{n_launch} launches in {len(groups)} groups; sum of group times {total_ms:.3f} ms per "
        f"chunk; the captured chunk replays in {statistics.median(ts):.3f} ms (median of 10).  "
        f"Top 25 by time per chunk:\n\n{rows}\n")
    log(f"wrote {path}: {n_launch} launches, {total_ms:.3f} ms summed, "
        f"{statistics.median(ts):.3f} ms per graph replay")


def batch_sweep(cfg, params, batches, out_path):
    """Chunk time and throughput at each batch size in ``batches`` (one engine
    each, graph replays, median of 10 after 3 warm-ups), with the engine's
    expert path and the ViT projections on the slab-blocked 256x256 GEMM, into
    ``out_path`` (markdown)."""
    from smolvla import layers
    from smolvla.params import smolvla_inputs
    from smolvla.pipeline import SmolVLAEngine
    v = cfg.vit
    L = ["# Chunk time against batch size (bench.py --batch-sweep)\n",
         "Command (repo root on the MI355X box): `python bench.py --batch-sweep "
         + " ".join(map(str, batches)) + "`\n",
         "One engine per batch size (seeded random-init bf16 weights, synthetic inputs resident "
         "in HBM); each chunk is one HIP-graph replay, median of 10 after 3 warm-ups, timed with "
         "HIP events on the engine's stream.  *ViT on 256x256*: the projections that "
         "`layers.vit_blocked_plan` puts on the slab-blocked 256x256 GEMM at that row count.  "
         "Boxes differ by up to +-15% in clock.\n",
         "| batch | expert | ViT on 256x256 | ms per chunk | chunks/s | TFLOP/s end to end |",
         "|---:|---|---|---:|---:|---:|"]
    for b in batches:
        eng = SmolVLAEngine(cfg, params, batch=b)
        eng.load_inputs(*smolvla_inputs(cfg, b, seed=1, device="cuda"))
        eng.capture()
        for _ in range(3):
            eng.step()
        ms = statistics.median(time_chunks(eng, 10))
        eng.check()
        plan = layers.vit_blocked_plan(v.hidden, v.inter, b * cfg.n_cameras * v.tokens)
        on = ", ".join(k for k, x in plan.items() if x) or "none"
        kind = "fused (one launch)" if eng.fx is not None else "layer by layer"
        L.append(f"| {b} | {kind} | {on} | {ms:.3f} | {b / ms * 1e3:.1f} | "
                 f"{chunk_flops(cfg, b) / (ms * 1e-3) / 1e12:.1f} |")
        log(f"batch {b}: {ms:.3f} ms per chunk, {b / ms * 1e3:.1f} chunks/s")
        del eng
        torch.cuda.empty_cache()
    pathlib.Path(out_path).write_text("\n".join(L) + "\n")
    log(f"wrote {out_path}")


def expert_phase_table(cfg, params, runs, out_path):
    """Per-phase timing of the batch-1 fused expert (``plan.stamps``: the
    team's first workgroup records the GPU's 100 MHz clock at every phase's
    start and at its own arrival) over ``runs`` eager launches, each on the
    chunk's own inputs; grouped by phase kind into ``out_path`` (markdown)."""
    import collections
    from smolvla.params import smolvla_inputs
    from smolvla.pipeline import SmolVLAEngine
    eng = SmolVLAEngine(cfg, params, batch=1)
    inp = smolvla_inputs(cfg, 1, seed=1, device="cuda")
    eng.run(*inp)                                   # prefix, cross K/V, a captured chunk
    fx = eng.fx
    kinds = fx.phase_kinds()
    per = []
    for _ in range(runs):
        eng.x_t.copy_(eng.in_noise.view(-1, cfg.action_dim))
        st = fx.phase_stamps().double() * 10.0 / 1e3     # 100 MHz ticks -> us
        per.append(st)
        if fx.status() != 0:
            raise SystemExit("fused expert failed during the phase timing")
    n = len(kinds)
    if per[0].shape[0] != n:
        raise SystemExit(f"phase count {per[0].shape[0]} != {n} named phases")
    span = statistics.median(float(s[-1, 1] - s[0, 0]) for s in per)
    groups = collections.OrderedDict()
    for i, k in enumerate(kinds):
        s2s = statistics.median(float((s[i + 1, 0] if i + 1 < n else s[i, 1]) - s[i, 0]) for s in per)
        own = statistics.median(float(s[i, 1] - s[i, 0]) for s in per)
        g = groups.setdefault(k, [0, 0.0, 0.0])
        g[0] += 1
        g[1] += s2s
        g[2] += own
    L = ["# Fused action expert, batch 1: time per phase kind\n",
         "Command (repo root on the MI355X box): `python bench.py --expert-phases "
         f"{runs}`\n",
         f"One launch runs {n} dependent phases.  The team's first workgroup records the GPU's "
         "100 MHz clock (`s_memrealtime`) when each phase starts (its wait for the previous "
         "phase done) and after its own arrival (its units' stores acknowledged, its count "
         "added): *start to start* is the phase's share of the launch's critical path, "
         "*own unit* the first workgroup's work inside it (the rest is the hand-off: the last "
         f"unit's arrival and the poll round trip).  Medians over {runs} eager launches on the "
         "chunk's own inputs; stamps add two stores per phase to that workgroup.\n",
         f"Launch span (first start to last arrival): {span / 1e3:.3f} ms, "
         f"{span / n:.2f} us per phase.\n",
         "| phase kind | phases | us start to start (mean) | us own unit (mean) | ms per launch | % |",
         "|---|---:|---:|---:|---:|---:|"]
    tot = sum(g[1] for g in groups.values())
    for k, (c, s2s, own) in sorted(groups.items(), key=lambda kv: -kv[1][1]):
        L.append(f"| {k} | {c} | {s2s / c:.2f} | {own / c:.2f} | {s2s / 1e3:.3f} | "
                 f"{100 * s2s / tot:.1f} |")
    pathlib.Path(out_path).write_text("\n".join(L) + "\n")
    log(f"wrote {out_path}: {n} phases, span {span / 1e3:.3f} ms")


def profile_chunks(cfg, params, batch, calls_out, eager_only):
    """Profiler entry point (``--profile-chunks``): the libsvla calls of one
    chunk at ``batch`` (with their work model and, unless ``eager_only``, the
    census's isolated replay times) written to ``calls_out``; then the chunk
    once more, as the last work of the process: three graph replays, or
    (``eager_only``, for counter runs) one eager chunk."""
    from smolvla import census
    from smolvla.params import smolvla_inputs
    from smolvla.pipeline import SmolVLAEngine
    eng = SmolVLAEngine(cfg, params, batch=batch, use_graph=False)
    eng.load_inputs(*smolvla_inputs(cfg, batch, seed=1, device="cuda"))
    eng.step()
    calls = census.record_chunk(eng)
    iso = {}
    if not eager_only:
        for g in census.time_groups(census.group_calls(calls, cfg, batch)):
            iso[g.label] = g.us
    pathlib.Path(calls_out).write_text(json.dumps(
        {"batch": batch, "calls": census.call_list(calls, cfg, batch), "iso_us": iso}))
    if eager_only:
        eng.step()
    else:
        eng.use_graph = True
        eng.capture()
        for _ in range(3):
            eng.step()
    torch.cuda.synchronize()
    eng.check()
    log(f"profile chunks at batch {batch}: {len(calls)} calls per chunk")


def profile_summary(calls_json, trace_csv, pmc_csvs, out_md, trace_cmd, pmc_cmds):
    """profiles/kernel_table_inchunk_bs<B>.md from a kernel-trace run and the
    counter runs of ``--profile-chunks``."""
    import csv
    from smolvla import census
    rec = json.loads(pathlib.Path(calls_json).read_text())
    calls = [tuple(c) for c in rec["calls"]]
    trace = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    pmc = [list(csv.DictReader(open(p))) for p in pmc_csvs]
    rows, total_ms, n = census.profile_table(calls, rec["iso_us"], trace, pmc, rec["batch"])
    cmds = "\n".join([trace_cmd] + pmc_cmds)
    pathlib.Path(out_md).write_text(
        f"# In-chunk kernel profile: one SmolVLA chunk at batch {rec['batch']}\n\n"
        f"Commands (repo root on the MI355X box, `cd /tmp && export TMPDIR=/tmp` first, `R` = repo "
        f"root; the counter runs one pass each):\n\n```\n{cmds}\n```\n\n"
        f"The {n} library dispatches of the last graph-replayed chunk of the kernel trace are matched, "
        f"in order, to the chunk's {len(calls)} libsvla calls (kernel families checked call by call) and "
        f"grouped as the census groups them (entry point, shape, epilogue).  *isolated us*: the census's "
        f"replay of the group alone in a graph; *in-chunk us*: the group's launches inside the replayed "
        f"chunk (rocprofv3 kernel trace).  Peak fraction from the in-chunk time (2.5 PFLOP/s bf16 MFMA or "
        f"8 TB/s HBM).  Counters per dispatch, averaged over the group's launches in one eager chunk of "
        f"each counter run: *MFMA busy* = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs); "
        f"*issuing* / *waiting* = SQ_ACTIVE_INST_ANY / SQ_WAIT_ANY over SQ_WAVE_CYCLES; *L2 hit* = "
        f"TCC_HIT / (TCC_HIT + TCC_MISS); *fetched / algorithmic* = FETCH_SIZE x 1024 x "
        f"{census.FETCH_SCALE:g} (the copy calibration) over the group's algorithmic bytes.\n\n"
        f"Sum of in-chunk kernel time: {total_ms:.3f} ms per chunk.  Top 30 groups by time:\n\n{rows}\n")
    log(f"wrote {out_md}: {n} dispatches, {total_ms:.3f} ms of kernel time")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--latency-chunks", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-latency", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-config (BASELINE configs 0-3, batch 1) lines")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the dominant kernel and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="turn the two --traffic-probe counter CSVs into the committed record")
    ap.add_argument("--profile-chunks", type=int, metavar="BATCH",
                    help="profiler entry point: write one chunk's call list to --calls-out, then "
                         "replay the chunk (run under rocprofv3)")
    ap.add_argument("--calls-out", default="chunk_calls.json")
    ap.add_argument("--eager-only", action="store_true",
                    help="with --profile-chunks: end with one eager chunk (counter runs)")
    ap.add_argument("--profile-summary", nargs="+", metavar="CSV",
                    help="CALLS_JSON TRACE_CSV [PMC_CSV ...]: write --out from a --profile-chunks "
                         "kernel trace and its counter runs")
    ap.add_argument("--out", default=None)
    ap.add_argument("--trace-cmd", default="")
    ap.add_argument("--pmc-cmd", action="append", default=[])
    ap.add_argument("--expert-phases", type=int, metavar="RUNS",
                    help="only write the batch-1 fused expert's per-phase timing (RUNS eager "
                         "launches) to profiles/expert_phases_bs1.md")
    ap.add_argument("--batch-sweep", type=int, nargs="+", metavar="BATCH",
                    help="chunk time and chunks/s at each batch size -> profiles/batch_sweep.md")
    ap.add_argument("--kernel-table", type=int, metavar="BATCH",
                    help="only write the per-kernel census table of one chunk at this batch "
                         "to profiles/kernel_table_bs<BATCH>.md")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build runs on a single GPU "
              "(data-parallel sharding over samples is design-only); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    from smolvla.config import SmolVLAConfig
    from smolvla.params import smolvla_inputs, smolvla_params
    from smolvla.pipeline import SmolVLAEngine

    cfg = SmolVLAConfig()
    if args.traffic_probe:
        traffic_probe(cfg, args.batch)
        return
    if args.traffic_summary:
        v = cfg.vit
        traffic_summary(*args.traffic_summary,
                        (args.batch * cfg.n_cameras * v.tokens, v.inter, v.hidden))
        return
    if args.profile_summary:
        a = args.profile_summary
        profile_summary(a[0], a[1], a[2:], args.out, args.trace_cmd, args.pmc_cmd)
        return
    log("generating seeded random-init bf16 weights")
    params = smolvla_params(cfg, seed=0)
    if args.profile_chunks:
        profile_chunks(cfg, params, args.profile_chunks, args.calls_out, args.eager_only)
        return
    if args.expert_phases:
        expert_phase_table(cfg, params, args.expert_phases,
                           args.out or str(ROOT / "profiles" / "expert_phases_bs1.md"))
        return
    if args.kernel_table:
        write_kernel_table(cfg, params, args.kernel_table)
        return
    if args.batch_sweep:
        batch_sweep(cfg, params, args.batch_sweep,
                    args.out or str(ROOT / "profiles" / "batch_sweep.md"))
        return
    B = args.batch
    log(f"preparing engine at batch {B}")
    eng = SmolVLAEngine(cfg, params, batch=B)
    inp = smolvla_inputs(cfg, B, seed=1, device="cuda")
    eng.load_inputs(*inp)
    eng.capture()
    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        eng.step()
    torch.cuda.synchronize()
    log(f"timing {args.steps} chunks at batch {B}")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_step = el / args.steps * 1e3
    value = B * args.steps / el
    flops = chunk_flops(cfg, B)
    log(f"batch {B}: {ms_step:.2f} ms/chunk-batch, {value:.1f} chunks/s, "
        f"{flops / (ms_step * 1e-3) / 1e12:.1f} TFLOP/s end to end")
    # the timed replays' result (inputs unchanged since the first replay)
    timed_out = eng.x_t.view(B, cfg.chunk, cfg.action_dim)[0].clone()
    eng.check()
    roof, _ = dominant_roofline(eng)
    log(f"dominant kernel: {roof['kernel']}, {roof['avg_launch_us']} us/launch x "
        f"{roof['launches_per_chunk']}, {roof['achieved']} {roof['unit']}")
    del eng
    torch.cuda.empty_cache()

    # output check, outside every timed region: the timed engine's actions are
    # finite and sample 0 equals what the batch-1 engine (other kernels: the
    # fused expert, batch-1 tiles) computes from the same inputs
    e1 = SmolVLAEngine(cfg, params, batch=1)
    one = e1.run(*[t[:1] for t in inp])[0]
    check = {"finite": bool(torch.isfinite(timed_out).all().item()),
             "sample0_max_abs_vs_bs1_engine": round((one - timed_out).abs().max().item(), 5),
             "atol": OUTPUT_ATOL}
    log(f"output check: {check}")
    if not check["finite"] or check["sample0_max_abs_vs_bs1_engine"] > OUTPUT_ATOL:
        raise SystemExit(f"bench: the timed engine's actions fail the output check {check}")

    lat = None
    if not args.no_latency:
        log("latency engine at batch 1")
        e1.load_inputs(*smolvla_inputs(cfg, 1, seed=2, device="cuda"))
        e1.capture()
        time_chunks(e1, 10)
        ts = time_chunks(e1, args.latency_chunks)
        med = statistics.median(ts)
        floor_us, bound, fl, by = chunk_floor(cfg, params, 1)
        lat = {"ms_per_chunk_median": round(med, 3),
               "ms_per_chunk_min": round(min(ts), 3), "chunks": len(ts), "batch": 1,
               "tflops_end_to_end": round(fl / (med * 1e-3) / 1e12, 1),
               "roofline": {"bound": bound, "floor_us": round(floor_us, 1),
                            "achieved_tflops": round(fl / (med * 1e-3) / 1e12, 1),
                            "achieved_gbs": round(by / (med * 1e-3) / 1e9, 1),
                            "flops": fl, "bytes": by, "frac": round(floor_us / (med * 1e3), 4)}}
        e1.check()
        log(f"batch 1 latency: median {lat['ms_per_chunk_median']} ms")
    gpu_cfg = None if args.no_configs else gpu_configs(cfg, params, e1)
    del e1
    torch.cuda.empty_cache()

    cpu = None
    cpu_cfg, threads = None, None
    if not args.no_cpu:
        log(f"CPU oracle baseline (~{args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(cfg, params, args.cpu_seconds)
        log(f"CPU: {cpu['value']} chunks/s on {cpu['cores']} threads")
        if gpu_cfg:
            cpu_cfg, threads = cpu_configs(cfg, params)
    configs = config_lines(cfg, params, gpu_cfg, cpu_cfg, threads) if gpu_cfg else None

    line = {
        "metric": "ms per 50-step action chunk @bs1; chunks/s @bs32; % MFMA/HBM roofline",
        "value": round(value, 2), "unit": "chunks/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded random-init bf16 weights; pixels U(-1,1), token ids, "
                "state and noise N(0,1))",
        "config": {"workload": "BASELINE config 4: full SmolVLA chunk (3 cams 512x512, "
                               "48 lang tokens, 241-token prefix x16 layers, 10 Euler steps "
                               "x16 expert layers)", "global_batch": B, "chunk": cfg.chunk,
                   "parallelism": "single GPU"},
        "output_check": check,
        "latency_bs1": lat,
        "configs_bs1": configs,
        "tflops_end_to_end": round(flops / (ms_step * 1e-3) / 1e12, 1),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
