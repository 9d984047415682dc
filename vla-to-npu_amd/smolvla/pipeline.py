"""Full SmolVLA inference engine on one MI355X.

One *chunk* per sample: 3 camera images -> SigLIP ViT (12 blocks) -> pixel-
shuffle connector -> [images | language | state] prefix (241 tokens) through
16 decoder layers, keeping every layer's K/V -> 10 Euler flow-matching steps of
the 16-layer action expert -> a 50x32 action chunk.

Composition follows the reference pipeline (vla/vla.py:228-338,
``joint_transformer`` vla/vla.py:194-212: expert layer i self-attends when
``i % 2 == 0`` and cross-attends to VLM layer i's K/V otherwise) extended to
the target configuration (3 cameras, 241-token prefix with a prefix-LM mask,
flow matching).  Because the prefix does not depend on the expert, all 16
prefix layers run first and their K/V stay resident; the cross-layer K/V
projections are hoisted out of the 10 Euler steps.

Everything after the input copy is launches of ``libsvla.so`` kernels on one
stream, captured once into a HIP graph (``torch.cuda.CUDAGraph``) and replayed
per chunk.  All buffers are allocated up front for the engine's batch size.
"""

from __future__ import annotations

import math

import torch

from . import layers, ops
from .config import SmolVLAConfig, resolve_eps

BF16 = torch.bfloat16
F32 = torch.float32


# the fused (one persistent launch) expert is used up to this many rows
# (batch * chunk): one 64-row block per GEMM unit
FUSED_EXPERT_MAX_ROWS = 64


class SmolVLAEngine:
    """``fused_expert``: run the 10-step action expert as one persistent
    launch (``ops.FusedExpert``) instead of ~840 layer-by-layer launches;
    default: when batch * chunk <= FUSED_EXPERT_MAX_ROWS (batch 1).
    ``expert_team_xcd``: the fused expert's CUs (-1: all; 0..7: one XCD)."""

    def __init__(self, cfg: SmolVLAConfig, params, batch: int, device="cuda", use_graph=True,
                 fused_expert=None, expert_team_xcd=-1):
        self.cfg = cfg
        self.B = batch
        self.device = torch.device(device)
        self.use_graph = use_graph
        self.graph = None
        if fused_expert is None:
            fused_expert = batch * cfg.chunk <= FUSED_EXPERT_MAX_ROWS
        self.fused_expert = fused_expert
        self.expert_team_xcd = expert_team_xcd
        self.fx = None
        with torch.cuda.device(self.device):
            ops.init()
            self._prepare(params)
            self._alloc()

    # ------------------------------------------------------------ set-up ---
    def _prepare(self, P):
        cfg, dev = self.cfg, self.device
        v, d, e = cfg.vit, cfg.decoder, cfg.expert
        pd = lambda t: t.to(device=dev, dtype=BF16).contiguous()  # noqa: E731
        self.patch_w = pd(P["patch"]["kernel"]).reshape(v.hidden, -1)
        self.patch_b = pd(P["patch"]["bias"])
        self.pos_emb = pd(P["patch"]["pos_emb"])
        vit_rows = self.B * cfg.n_cameras * v.tokens
        self.vit = [layers.prep_vit(lp, dev, rows=vit_rows) for lp in P["vit"]]
        self.conn_w = ops.pack_weight(pd(P["connector"]["W"]))
        self.embed_table = pd(P["embed"])
        self.state_w = ops.pack_weight(pd(P["state"]["W"]))
        self.prefix = [layers.prep_decoder(lp, dev) for lp in P["prefix"]]
        self.expert = [layers.prep_cross(lp, dev) if cfg.is_cross(i) else layers.prep_decoder(lp, dev)
                       for i, lp in enumerate(P["expert"])]
        io = P["expert_io"]
        H = e.hidden
        self.w_ain = ops.pack_weight(pd(io["W_action_in"]))
        self.b_ain = pd(io["b_action_in"])
        w_tin = pd(io["W_time_in"])
        self.w_tin_a = ops.pack_weight(w_tin[:H].contiguous())
        self.w_tin_t = ops.pack_weight(w_tin[H:].contiguous())
        self.b_tin = pd(io["b_time_in"])
        self.w_tout = ops.pack_weight(pd(io["W_time_out"]))
        self.b_tout = pd(io["b_time_out"])
        self.n_exp = pd(io["W_exp_norm"])
        self.w_aout = ops.pack_weight(pd(io["W_action_out"]))
        self.rope_prefix = layers.Rope.make(cfg.prefix_len, d.head_dim, d.rope_theta, dev)
        self.rope_expert = layers.Rope.make(cfg.chunk, e.head_dim, e.rope_theta, dev)
        torch.cuda.synchronize(dev)

    def _alloc(self):
        cfg, dev, B = self.cfg, self.device, self.B
        v, d, e = cfg.vit, cfg.decoder, cfg.expert
        z = lambda *s, dt=BF16: torch.zeros(*s, dtype=dt, device=dev)  # noqa: E731
        nimg = B * cfg.n_cameras
        # inputs (static: the graph reads them)
        self.in_images = z(nimg, v.channels, v.image, v.image)
        self.in_ids = torch.zeros(B, cfg.lang_tokens, dtype=torch.int64, device=dev)
        self.in_state = z(B, cfg.state_dim, dt=F32)
        self.in_noise = z(B, cfg.chunk, cfg.action_dim, dt=F32)
        # vision
        self.vit_x = z(nimg * v.tokens, v.hidden)
        self.vbufs = layers.Buffers(dev)
        # prefix
        L = cfg.prefix_len
        self.prefix_x = z(B * L, d.hidden)
        self.state_bf = z(B, cfg.state_dim)
        self.kv = [z(B * L, d.q_dim + 2 * d.kv_dim) for _ in range(cfg.prefix_layers)]
        self.pbufs = layers.Buffers(dev)
        # expert
        # projected cross K | V of a layer side by side in one buffer (one GEMM
        # projects both, layers.cross_kv)
        self.cross = {}
        for i in range(cfg.expert_layers):
            if cfg.is_cross(i):
                ckv = z(B * L, 2 * e.kv_dim)
                self.cross[i] = (ckv[:, :e.kv_dim], ckv[:, e.kv_dim:])
        M = B * cfg.chunk
        self.x_t = z(M, cfg.action_dim, dt=F32)
        self.x_bf = z(M, cfg.action_dim)
        self.temb = z(cfg.num_steps, e.hidden)
        self.tbias = z(cfg.num_steps, e.hidden, dt=F32)
        self.a_emb = z(M, e.hidden)
        self.h_time = z(M, e.hidden)
        self.ex = z(M, e.hidden)
        self.ebufs = layers.Buffers(dev)
        # the time part of the action-time MLP input depends only on the
        # weights and the fixed Euler schedule: computed once, like the RoPE
        # tables, not per chunk
        self.time_bias(self.schedule())
        if self.fused_expert:
            io = dict(w_ain=self.w_ain, b_ain=self.b_ain, w_tin_a=self.w_tin_a,
                      w_tout=self.w_tout, b_tout=self.b_tout, n_exp=self.n_exp,
                      w_aout=self.w_aout)
            self.fx = ops.FusedExpert(cfg, self.expert, self.cross, io, self.rope_expert,
                                      self.tbias, self.x_t, B, -1.0 / cfg.num_steps,
                                      team_xcd=self.expert_team_xcd)
        # materialise every lazily-named buffer before any capture
        self._forward()
        torch.cuda.synchronize(dev)

    # ----------------------------------------------------------- stages ---
    def vision(self):
        cfg = self.cfg
        v = cfg.vit
        nimg = self.B * cfg.n_cameras
        ops.patch_embed(self.in_images, self.patch_w, self.patch_b, self.pos_emb, v.patch,
                        out=self.vit_x)
        for P in self.vit:
            layers.vit_layer(self.vit_x, P, v, nimg, v.tokens, self.vbufs)

    def build_prefix(self):
        cfg = self.cfg
        d = cfg.decoder
        L = cfg.prefix_len
        nimg = self.B * cfg.n_cameras
        img_rows = cfg.n_cameras * cfg.image_tokens
        ops.connector(self.vit_x.view(nimg, cfg.vit.tokens, cfg.vit.hidden), self.conn_w,
                      cfg.pixel_shuffle, out=self.prefix_x, rows_per_sample=img_rows,
                      sample_stride=L)
        ops.embed(self.in_ids, self.embed_table, math.sqrt(d.hidden), self.prefix_x[img_rows:],
                  per_sample=cfg.lang_tokens, out_bs=L * d.hidden)
        ops.f32_to_bf16(self.in_state, out=self.state_bf)
        st_rows = self.prefix_x.view(self.B, L, d.hidden)[:, L - 1, :]
        ops.linear(self.state_bf, self.state_w, out=st_rows)

    def run_prefix(self):
        cfg = self.cfg
        for P, kv in zip(self.prefix, self.kv):
            layers.decoder_layer(self.prefix_x, P, cfg.decoder, self.B, cfg.prefix_len,
                                 self.rope_prefix, cfg.prefix_mask, cfg.prefix_bidir_len,
                                 self.pbufs, qkv_out=kv)

    def project_cross(self):
        d = self.cfg.decoder
        qd, kvd = d.q_dim, d.kv_dim
        for i, (ck, cv) in self.cross.items():
            kv = self.kv[i]
            layers.cross_kv(kv[:, qd:qd + kvd], kv[:, qd + kvd:], self.expert[i], out_k=ck,
                            out_v=cv)

    def schedule(self):
        """Euler times t_s = 1, 1 + dt, ... (dt = -1 / num_steps)."""
        dt = -1.0 / self.cfg.num_steps
        ts, t = [], 1.0
        for _ in range(self.cfg.num_steps):
            ts.append(t)
            t = t + dt
        return ts

    def time_bias(self, ts):
        """Time part of the action-time MLP input for every Euler step, hoisted
        out of the chunk (it depends on t only, and the schedule is fixed; the
        engine computes it once at set-up): tbias[s] = temb(t_s) @ W_time_in[H:]
        + b_time_in, kept in fp32 so that the per-step GEMM rounds once as the
        concatenated projection does."""
        e = self.cfg.expert
        for s, t in enumerate(ts):
            ops.time_embedding(t, e.hidden, out=self.temb[s])
        ops.linear(self.temb, self.w_tin_t, bias=self.b_tin, out=self.tbias, out_f32=True)

    def expert_step(self, s, dt):
        cfg = self.cfg
        e = cfg.expert
        B, L, Lc = self.B, cfg.chunk, cfg.prefix_len
        # action / time embedding
        ops.linear(self.x_bf, self.w_ain, bias=self.b_ain, out=self.a_emb)
        ops.linear(self.a_emb, self.w_tin_a, bias_f32=self.tbias[s], act="silu",
                   out=self.h_time)
        ops.linear(self.h_time, self.w_tout, bias=self.b_tout, out=self.ex)
        for i, P in enumerate(self.expert):
            if cfg.is_cross(i):
                ck, cv = self.cross[i]
                layers.cross_layer(self.ex, ck, cv, P, e, B, L, Lc, self.rope_expert,
                                   self.ebufs)
            else:
                layers.decoder_layer(self.ex, P, e, B, L, self.rope_expert, "causal", 0,
                                     self.ebufs)
        # final expert RMSNorm (one rounding, as torch's) then action_out + Euler
        # (vla/vla.py:218-222)
        h = ops.rmsnorm(self.ex, self.n_exp, resolve_eps(e.rms_eps),
                        out=self.ebufs.get("xn_out", B * L, e.hidden))
        ops.action_out_euler(h, self.w_aout, self.x_t, dt, x_bf16=self.x_bf)

    def _forward(self):
        cfg = self.cfg
        self.vision()
        self.build_prefix()
        self.run_prefix()
        self.project_cross()
        self.x_t.copy_(self.in_noise.view(-1, cfg.action_dim))
        if self.fx is not None:
            self.fx.run()
            return
        ops.f32_to_bf16(self.x_t, out=self.x_bf)
        dt = -1.0 / cfg.num_steps
        for s in range(cfg.num_steps):
            self.expert_step(s, dt)

    # ------------------------------------------------------------ public ---
    def load_inputs(self, images, lang_ids, state, noise):
        B, cfg = self.B, self.cfg
        self.in_images.copy_(images.reshape(B * cfg.n_cameras, *images.shape[2:]))
        self.in_ids.copy_(lang_ids)
        self.in_state.copy_(state)
        self.in_noise.copy_(noise)

    def capture(self):
        """Record one whole chunk into a HIP graph (after a warm-up run)."""
        with torch.cuda.device(self.device):
            s = torch.cuda.Stream(device=self.device)
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                self._forward()
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize(self.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._forward()
            torch.cuda.synchronize(self.device)
            self.graph = g

    def step(self):
        """Run one chunk on the inputs already in the static input buffers."""
        if self.use_graph:
            if self.graph is None:
                self.capture()
            self.graph.replay()
        else:
            self._forward()

    def check(self):
        """Raise if the last chunk's fused expert gave up (its status word is
        non-zero: a wait timed out, e.g. because other work held CUs the
        persistent launch needed, or its XCD team did not form).  Such a
        chunk's actions are NaN-filled by the kernel as well.  Synchronous."""
        if self.fx is None:
            return
        st = self.fx.status()
        if st != 0:
            what = {1: "a phase wait timed out", 2: "the XCD team did not form"}.get(st, "?")
            raise RuntimeError(f"fused action expert failed (status {st}: {what}); the "
                               "chunk's actions are invalid")

    def run(self, images, lang_ids, state, noise):
        """images ``[B, cams, 3, H, W]`` bf16, lang_ids ``[B, 48]``, state
        ``[B, 32]``, noise ``[B, 50, 32]`` fp32 -> actions ``[B, 50, 32]`` fp32.
        Raises if the fused expert reports a failure (:meth:`check`)."""
        with torch.cuda.device(self.device):
            self.load_inputs(images, lang_ids, state, noise)
            self.step()
            out = self.x_t.view(self.B, self.cfg.chunk, self.cfg.action_dim).clone()
            self.check()
            return out

    # intermediate views (tests)
    def prefix_view(self):
        return self.prefix_x.view(self.B, self.cfg.prefix_len, -1)
