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
  roofline     the dominant kernel (ViT MLP up-projection GEMM, bf16 MFMA):
               algorithmic FLOPs / average launch time from HIP events on its
               stream, against the 2.5 PFLOP/s dense bf16 peak
  cpu_baseline the CPU oracle (PyTorch bf16 restatement of the reference
               modules) timed on this host's cores on a bounded sample
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


def _up_proj_launcher(cfg, M, x, w_packed, bias, wide):
    """The ViT MLP up-projection exactly as the engine launches it at this
    row count: on the 256x256 kernel with slab-blocked activations (the
    LayerNorm writes them so), weights and output when ``wide``
    (``layers.vit_wide_ok``), else through ``ops.linear``."""
    from smolvla import ops
    v = cfg.vit
    if wide:
        xb = ops.slab_block(x)
        wb = ops.slab_block(w_packed)
        out = torch.empty(v.inter // 32, M, 32, device="cuda", dtype=torch.bfloat16)
        lay = ops.LAYOUT_A_BLOCKED | ops.LAYOUT_W_BLOCKED | ops.LAYOUT_C_BLOCKED
        return lambda: ops.linear_wide(xb, wb, M, v.inter, v.hidden, bias=bias,
                                       act="gelu_" + v.gelu, out=out, layout=lay)
    out = torch.empty(M, v.inter, device="cuda", dtype=torch.bfloat16)
    return lambda: ops.linear(x, w_packed, bias=bias, act="gelu_" + v.gelu, out=out)


def dominant_kernel_roofline(eng, iters):
    """The ViT MLP up-projection (GEMM 96k x 3072 x 768 at batch 32 with the
    bias + tanh-GELU epilogue; the only GEMM instantiated with GELU), launched
    as the engine launches it, `iters` times back-to-back on the current
    stream between two HIP events."""
    from smolvla import layers
    cfg = eng.cfg
    v = cfg.vit
    P = eng.vit[0]
    M = eng.vit_x.shape[0]
    x = eng.vbufs.get("vh", M, v.hidden)
    wide = layers.vit_wide_ok(v, M)
    run = _up_proj_launcher(cfg, M, x, P["wup"], P["bup"], wide)
    for _ in range(3):
        run()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        run()
    b.record()
    b.synchronize()
    avg_ms = a.elapsed_time(b) / iters
    flops = 2.0 * M * v.inter * v.hidden
    achieved = flops / (avg_ms * 1e-3) / 1e12
    hbm_bytes = 2.0 * (M * v.hidden + v.inter * v.hidden + M * v.inter + v.inter)
    tr = load_traffic()
    traffic = tr.get("bytes_per_launch") if tr and tr.get("shape") == [M, v.inter, v.hidden] else None
    from smolvla import _lib
    tile = _lib.load().svla_gemm_tile_choice(M, v.inter, v.hidden, 1)
    kname = {8: "gemm_wide_kernel<0, false, 0, 1, false> (persistent 256x256 tile, 5-stage "
                "LDS-DMA ring, LDS-staged bias + tanh-GELU epilogue, streaming stores" +
                (", slab-blocked activations, weights and output)" if wide else ")"),
             7: "gemm_pipe_kernel<128, 128, 0, false, 0, 1> (128x128 LDS-DMA pipeline, "
                "bias + tanh-GELU epilogue)"}.get(tile, f"GEMM tile configuration {tile}")
    return {
        "kernel": kname + ": ViT MLP up-projection",
        "shape": [M, v.inter, v.hidden],
        "bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
        "avg_launch_us": round(avg_ms * 1e3, 2), "algorithmic_bytes": hbm_bytes,
        "traffic": traffic,
    }


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
    from smolvla import layers
    run = _up_proj_launcher(cfg, M, x, w, b, layers.vit_wide_ok(v, M))
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
            "kind": "port",
            "sample": f"{n} full bs=1 chunks (3x512^2 cameras, 241-token prefix, 10 Euler "
                      f"steps) in {el:.1f} s, torch {torch.__version__} bf16 on CPU",
            "ms_per_chunk": round(el / n * 1e3, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--latency-chunks", type=int, default=50)
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-latency", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the dominant kernel and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="turn the two --traffic-probe counter CSVs into the committed record")
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
    log("generating seeded random-init bf16 weights")
    params = smolvla_params(cfg, seed=0)
    B = args.batch
    log(f"preparing engine at batch {B}")
    eng = SmolVLAEngine(cfg, params, batch=B)
    eng.load_inputs(*smolvla_inputs(cfg, B, seed=1, device="cuda"))
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
    roof = dominant_kernel_roofline(eng, args.kernel_iters)
    log(f"dominant kernel: {roof['avg_launch_us']} us/launch, {roof['achieved']} TFLOP/s")
    del eng
    torch.cuda.empty_cache()

    lat = None
    if not args.no_latency:
        log("latency engine at batch 1")
        e1 = SmolVLAEngine(cfg, params, batch=1)
        e1.load_inputs(*smolvla_inputs(cfg, 1, seed=2, device="cuda"))
        e1.capture()
        time_chunks(e1, 10)
        ts = time_chunks(e1, args.latency_chunks)
        lat = {"ms_per_chunk_median": round(statistics.median(ts), 3),
               "ms_per_chunk_min": round(min(ts), 3), "chunks": len(ts), "batch": 1,
               "tflops_end_to_end": round(chunk_flops(cfg, 1) / (statistics.median(ts) * 1e-3)
                                          / 1e12, 1)}
        log(f"batch 1 latency: median {lat['ms_per_chunk_median']} ms")
        del e1
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log(f"CPU oracle baseline (~{args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(cfg, params, args.cpu_seconds)
        log(f"CPU: {cpu['value']} chunks/s on {cpu['cores']} threads")

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
        "latency_bs1": lat,
        "tflops_end_to_end": round(flops / (ms_step * 1e-3) / 1e12, 1),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
