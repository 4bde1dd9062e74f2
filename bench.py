#!/usr/bin/env python3
"""Benchmark of the VASC sparse global-attention path on one MI355X.

Headline (the metric's configuration): frames/s of
the VGGT-shaped aggregator forward (24 frame + 24 global blocks, dim 1024,
16 heads, MLP 4096, random-init bf16) on 32 frames of 392x518 uniform noise
(33 312 global tokens), mode vasc at sparsity 0.75 with the structural
layer-budget profile. One step = one aggregator forward; ``value`` = 32 /
forward seconds. Beside it:

* the global layer in the reference's timer scope (qkv, layout, sparse op,
  restore, proj; median over the timed forwards) and the same for dense;
* the roofline of the dominant kernel, the block-sparse attention launch of
  the global layers, timed with hipEvents around each launch inside the
  timed forwards;
* the 24-layer sparse op alone on synthetic Q/K/V (pool + pooled softmax,
  VASC selection with the cross-layer ledger, V pack, attention) with
  per-kernel HBM rates and the dense-attention comparison;
* the CPU baseline (torch fp32 restatements of the reference's dense and
  topk paths on this host's cores).

Prints one JSON line (the driver's contract). Progress goes to stderr.
Other workloads: ``--workload c3`` (128 frames, s=0.875), ``c4`` (the
Pi3-shaped decoder at 64 frames), ``c5`` (kernel microbenchmarks);
``--probe`` runs untimed programs for rocprofv3 counter passes.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import torch

METRIC = "sparse global-attn layer ms + eff. TFLOP/s @75% sparsity, 32 frames; frames/s"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


TRAFFIC_SUMMARY = "profiles/traffic_c2_forward.md"


def traffic_bytes():
    """HBM bytes per attention launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary of this workload (calibrated against a plain copy)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_SUMMARY)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("attention_traffic_bytes_per_launch:"):
                    return float(line.split(":")[1])
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synthetic_layer(N: int, P: int, S: int, H: int, D: int, seed: int, device):
    """Q (patch only), K, V in [patch; special] order: N(0,1) plus a per-frame
    rank-8 component of scale 0.5 (the input recipe of the C1 configuration)."""
    g = torch.Generator(device=device).manual_seed(seed)
    out = []
    for _ in range(3):
        x = torch.randn(1, H, N, P, D, device=device, generator=g)
        u = torch.randn(1, H, N, P, 8, device=device, generator=g)
        w = torch.randn(1, H, N, 8, D, device=device, generator=g)
        x = x + 0.5 * (u @ w) / math.sqrt(8)
        patch = x[:, :, :, S:].reshape(1, H, N * (P - S), D)
        special = x[:, :, :, :S].reshape(1, H, N * S, D)
        out.append(torch.cat([patch, special], dim=2).to(torch.bfloat16).contiguous())
        del x, u, w
    q, k, v = out
    return q[:, :, : N * (P - S)].contiguous(), k, v


class Timer:
    """hipEvent pairs recorded on the current stream, summed per label."""

    def __init__(self, enabled: bool = True):
        self.enabled = enabled
        self.events: dict[str, list] = {}
        self._open = None

    def start(self, label):
        if self.enabled:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self._open = (label, ev)

    def stop(self):
        if self.enabled:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            label, a = self._open
            self.events.setdefault(label, []).append((a, ev))

    def totals_ms(self) -> dict:
        return {k: sum(a.elapsed_time(b) for a, b in v) for k, v in self.events.items()}

    def counts(self) -> dict:
        return {k: len(v) for k, v in self.events.items()}


def run_step(layers, ratios, ledger, timer, keep=None):
    """One step: the sparse op of every layer, ledger cleared first."""
    from vasc_amd import ops, pipeline
    ledger.clear()
    for li, (q, k, v) in enumerate(layers):
        n_patch = q.shape[2]
        plan = pipeline.LayerPlan.make(n_patch, k.shape[2])
        timer.start("pool")
        pq, pk, _, iota = ops.pool_qkv(q, k[:, :, :n_patch], v[:, :, :n_patch])
        timer.stop()
        timer.start("pooled_softmax")
        prob = ops.pooled_softmax(pq, pk)
        timer.stop()
        timer.start("select")
        sel = pipeline.select_layer(prob, iota, plan, mode="vasc", sparse_ratio=ratios[li],
                                    official_mask=True, ledger=ledger, layer_idx=li)
        timer.stop()
        timer.start("pack_v")
        vt = ops.pack_v(v)
        timer.stop()
        timer.start("attention")
        o = ops.block_sparse_attn(q, k, vt, sel["index"], sel["count"])
        timer.stop()
        if keep is not None:
            keep.append((sel["index"], sel["count"], o))


def attention_min_bytes(index, count, n_q, n_k, d):
    """Least HBM bytes one sparse-attention launch can move: Q read and O written
    once, plus every K block and packed V tile that some query block of the
    head selects, each read once (bf16). Returns (bytes, distinct key blocks
    listed per head)."""
    kb = -(-n_k // 64)
    width = index.shape[-1]
    valid = torch.arange(width, device=index.device) < count.unsqueeze(-1).long()
    idx = torch.where(valid, index.long(), kb).flatten(2)
    touched = torch.zeros(*idx.shape[:2], kb + 1, dtype=torch.bool, device=idx.device)
    touched.scatter_(2, idx, True)
    blocks = int(touched[..., :kb].sum().item())
    heads = index.shape[0] * index.shape[1]
    return heads * n_q * d * 2 * 2 + blocks * 64 * d * 2 * 2, blocks / heads


def attention_min_bytes_global(index, count, n_patch, n_total, n_special, H, d):
    """Least HBM bytes of one global-layer attention launch (B = 1): the patch
    and special queries read and their outputs written once, and every K
    block and packed V tile read once; the special queries attend to every
    key block, so each one is needed. Also returns the distinct key blocks
    the patch queries' lists name per head."""
    patch_only, listed = attention_min_bytes(index, count, n_patch, n_total, d)
    if n_special == 0:
        return patch_only, listed
    kb = -(-n_total // 64)
    return H * (n_patch + n_special) * d * 2 * 2 + H * kb * 64 * d * 2 * 2, listed


def hbm_bytes_per_launch(H, n_patch, n_total, d, listed_per_layer):
    """Algorithmic HBM bytes of one launch of each HBM-bound kernel (B = 1):
    every input read once and every output written once."""
    qb, kb = -(-n_patch // 128), -(-n_patch // 64)
    kbt = -(-n_total // 64)
    pooled = H * (qb + 2 * kb) * d * 2 + H * (-(-kb // 2)) * 4
    return {
        "pool": 3 * H * n_patch * d * 2 + pooled,
        "pooled_softmax": H * (qb + kb) * d * 2 + H * qb * kb * 4,
        "select": H * qb * kb * 4 + listed_per_layer * 4 + H * qb * 4,
        "pack_v": H * n_total * d * 2 + H * kbt * 64 * d * 2,
    }


def median_ms(fn, reps: int, rounds: int = 5) -> float:
    """Median over rounds of the mean time of ``reps`` back-to-back calls (hipEvents)."""
    times = []
    for _ in range(rounds):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) / reps)
    return statistics.median(times)


def c5_lists(T: int, H: int, rho: float, seed: int, device):
    """The C5 block lists: per query-block row k ~ Poisson(rho*Kb) clipped to
    [n_forced, Kb]; forced = key blocks holding tokens f*1041 + j (j < 5) of
    every frame f; the rest drawn uniformly without replacement; ascending."""
    qb, kb = T // 128, T // 64
    g = torch.Generator(device=device).manual_seed(seed)
    frames = -(-T // 1041)
    tok = (torch.arange(frames, device=device).view(-1, 1) * 1041 + torch.arange(5, device=device)).flatten()
    forced = torch.unique(tok[tok < T] // 64)
    nf = forced.numel()
    lam = torch.full((H, qb), rho * kb, device=device)
    k = torch.poisson(lam, generator=g).long().clamp(nf, kb)
    keys = torch.rand(H, qb, kb, device=device, generator=g)
    keys[:, :, forced] = -1.0  # forced blocks sort first
    order = torch.argsort(keys, dim=-1)
    pos = torch.arange(kb, device=device).view(1, 1, kb)
    chosen = torch.where(pos < k.unsqueeze(-1), order, kb)
    index = torch.sort(chosen, dim=-1).values.to(torch.int32).unsqueeze(0)
    del keys, order, chosen
    return index, k.to(torch.int32).unsqueeze(0)


def run_c5(dev) -> int:
    """C5: each kernel on randn bf16 [1,16,T,64] inputs, T in {16k, 64k, 256k};
    attention at densities 0.1 / 0.25 / 0.5 of Poisson block lists."""
    from vasc_amd import _lib, ops, pipeline
    H, D = 16, 64
    for T in (16384, 65536, 262144):
        g = torch.Generator(device=dev).manual_seed(T)
        q, k, v = (torch.randn(1, H, T, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
        qb, kb = T // 128, T // 64
        pq, pk, _, iota = ops.pool_qkv(q, k, v)
        prob = ops.pooled_softmax(pq, pk)
        topk = int(kb * 0.25)
        lines = []
        hbm = hbm_bytes_per_launch(H, T, T, D, 0)
        t = median_ms(lambda: ops.pool_qkv(q, k, v), 5)
        lines.append(("pool", t, hbm["pool"], None))
        t = median_ms(lambda: ops.pooled_softmax(pq, pk), 5)
        lines.append(("pooled_softmax", t, hbm["pooled_softmax"], None))
        for mode, name in ((_lib.MODE_TOPK, "select_topk"), (_lib.MODE_VASC, "select_vasc")):
            kw = dict(mode=mode, topk=topk)
            if mode == _lib.MODE_VASC:
                kw.update(innovation=iota, max_capacity=topk, workspace=ops.select_workspace(1, H, qb, kb, dev))
            sel = ops.select_blocks(prob, **kw)
            listed = int(sel["count"].sum().item())
            t = median_ms(lambda: ops.select_blocks(prob, **kw), 5)
            lines.append((name, t, H * qb * kb * 4 + listed * 4 + H * qb * 4, f"cap {topk} of {kb}"))
        # cdf-threshold counts (sort + sequential running sum per row); the
        # threshold array is built once so only the kernel is timed
        count = torch.empty(1, H, qb, device=dev, dtype=torch.int32)
        for thr in (0.5, 0.9):
            T_h = torch.full((H,), thr, dtype=torch.float32).add_(1e-5).to(dev)
            def cdf(T_h=T_h):
                _lib.call("vasc_cdf_counts", prob.data_ptr(), 1, H, qb, kb, T_h.data_ptr(), 0, 0, count.data_ptr(),
                          None, ops._stream())
            cdf()
            mean_n = float(count.float().mean().item())
            t = median_ms(cdf, 5)
            lines.append(("cdf_counts", t, H * qb * kb * 4 + H * qb * 4, f"threshold {thr}, mean count {mean_n:.1f}"))
        t = median_ms(lambda: ops.pack_v(v), 5)
        lines.append(("pack_v", t, hbm["pack_v"], None))
        for name, t, nbytes, note in lines:
            rec = {"workload": "C5", "kernel": name, "T": T, "ms": t, "bytes": nbytes,
                   "GB_s": nbytes / (t * 1e-3) / 1e9, "frac_of_hbm_peak": nbytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBS}
            if note:
                rec["note"] = note
            print(json.dumps(rec), flush=True)
        vt = ops.pack_v(v)
        for rho in (0.1, 0.25, 0.5):
            index, count = c5_lists(T, H, rho, seed=int(rho * 100) + T, device=dev)
            flops = pipeline.attention_flops((index, count), T, T, D)
            t = median_ms(lambda: ops.block_sparse_attn(q, k, vt, index, count), 3 if T > 65536 else 10)
            print(json.dumps({"workload": "C5", "kernel": "block_sparse_attn", "T": T, "density": rho,
                              "mean_blocks_per_row": float(count.float().mean().item()), "ms": t,
                              "flops": flops, "TFLOP_s": flops / (t * 1e-3) / 1e12,
                              "frac_of_mfma_peak": flops / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}), flush=True)
            del index, count
        t = median_ms(lambda: ops.dense_attn(q, k, vt), 1 if T > 65536 else 3, rounds=3)
        flops = 4.0 * D * H * T * T
        print(json.dumps({"workload": "C5", "kernel": "dense_attn", "T": T, "ms": t, "flops": flops,
                          "TFLOP_s": flops / (t * 1e-3) / 1e12,
                          "frac_of_mfma_peak": flops / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}), flush=True)
        del q, k, v, vt, prob, pq, pk, iota
        torch.cuda.empty_cache()
    return 0


class AttnLaunchEvents:
    """hipEvents around every ``ops.global_attn`` / ``ops.global_attn_tokens``
    launch (the sparse global layers' attention kernel) on the stream it is
    launched on, plus the lists of each layer's latest launch for its
    algorithmic flops."""

    _NAMES = ("global_attn", "global_attn_tokens")

    def __init__(self, layers: int):
        self.layers = layers
        self.events: list = []
        self.lists: dict = {}
        self.enabled = False

    def _wrap(self, orig):
        def timed(q_patch, q_special, k, vt, index, count, *args, **kw):
            if not self.enabled:
                return orig(q_patch, q_special, k, vt, index, count, *args, **kw)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            out = orig(q_patch, q_special, k, vt, index, count, *args, **kw)
            b.record()
            self.events.append((a, b))
            n_special = 0 if q_special is None else q_special.shape[2]
            self.lists[len(self.events) % self.layers] = (index, count, q_patch.shape[2], k.shape[2], n_special,
                                                          q_patch.shape[1], q_patch.shape[3])
            return out
        return timed

    def __enter__(self):
        from vasc_amd import ops
        self._ops = ops
        self._orig = {name: getattr(ops, name) for name in self._NAMES}
        for name, fn in self._orig.items():
            setattr(ops, name, self._wrap(fn))
        return self

    def __exit__(self, *exc):
        for name, fn in self._orig.items():
            setattr(self._ops, name, fn)

    def mean_ms(self) -> float:
        return statistics.fmean(a.elapsed_time(b) for a, b in self.events)

    def flops_per_launch(self) -> float:
        """Mean algorithmic flops of one launch: 4*d per (query, key) pair of
        the listed blocks, plus the special queries over every key."""
        from vasc_amd import pipeline
        tot = 0.0
        for index, count, n_patch, n_total, n_special, H, D in self.lists.values():
            tot += pipeline.attention_flops((index, count), n_patch, n_total, D)
            tot += 4.0 * D * H * n_special * n_total * index.shape[0]
        return tot / len(self.lists)


def build_aggregator(dev, seed: int = 0):
    from vasc_amd.aggregator import Aggregator
    torch.manual_seed(seed)
    with torch.device(dev):
        agg = Aggregator(dim=1024, depth=24, num_heads=16, mlp_ratio=4.0)
    return agg.to(torch.bfloat16).eval()


def _ModeEnv(backbone: str, mode: str):
    """The reference's SPARSE_VGGT_* switches of one release mode for a block."""
    from vasc_amd.launcher import use_mode
    return use_mode(backbone, mode)


def tune_gemms(enable: bool) -> None:
    """torch's TunableOp for the runners' hipBLASLt GEMMs: each GEMM shape is
    tuned (at most 30 trials or 200 ms) the first time it runs, in the dense
    warm-up forward, and the choice is reused by every later call. The
    results file goes to the temporary directory."""
    import tempfile
    import torch.cuda.tunable as tunable
    tunable.enable(enable)
    tunable.tuning_enable(enable)
    if enable:
        tunable.set_max_tuning_duration(200)
        tunable.set_max_tuning_iterations(30)
        tunable.set_filename(os.path.join(tempfile.gettempdir(), f"vasc_tunableop_{os.getpid()}.csv"))


def run_aggregator(dev, frames: int, ratios, steps: int, warmup: int, dense_reps: int = 3,
                   tune: bool = True) -> dict:
    """The VGGT-shaped aggregator (24 frame + 24 global blocks, dim 1024, 16
    heads, MLP 4096, random init bf16) on seeded uniform-noise images
    ``[1, frames, 3, 392, 518]``.

    * dense: every global block on the dense MFMA kernel (``dense_reps``
      forwards after one warm-up);
    * vasc with the per-layer ratios: ``warmup`` forwards, then exactly
      ``steps`` forwards timed between two synchronizations (the headline),
      with hipEvents around every global attention module (the reference's
      CudaAttentionTimer scope, eval_7scenes_sparse_vggt.py:1533-1574: qkv,
      layout, sparse op, restore, proj) and around every attention launch
      (the roofline's kernel).

    The block GEMMs (qkv, proj, fc1, fc2) run on hipBLASLt through torch;
    with ``tune`` torch's TunableOp picks their algorithms in the first
    (untimed) dense forward.
    """
    from vasc_amd import install
    agg = build_aggregator(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    images = torch.rand(1, frames, 3, 392, 518, device=dev, generator=g)
    layer_events: list = []

    def pre(mod, args, kwargs=None):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        layer_events.append([ev, None])

    def post(mod, args, out):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        layer_events[-1][1] = ev

    for blk in agg.global_blocks:
        blk.attn.register_forward_pre_hook(pre)
        blk.attn.register_forward_hook(post)
    L = len(agg.global_blocks)

    def forwards(n, timed):
        """n forwards; returns (total ms between synchronizations, per-forward
        global-layer ms)."""
        layer_events.clear()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        with torch.no_grad():
            for _ in range(n):
                agg(images)
        b.record()
        torch.cuda.synchronize()
        per_fwd = [sum(x.elapsed_time(y) for x, y in layer_events[i * L:(i + 1) * L]) for i in range(n)]
        return a.elapsed_time(b), per_fwd

    out = {}
    tune_gemms(tune)
    forwards(1, False)  # the warm-up forward tunes the GEMM shapes
    if tune:
        import torch.cuda.tunable as tunable
        tunable.tuning_enable(False)
        out["gemm_tuning"] = {"TunableOp": True, "tuned": len(tunable.get_results())}
    total, glob = forwards(dense_reps, True)
    out["dense"] = {"forward_ms": total / dense_reps, "frames_per_s": frames / (total / dense_reps * 1e-3),
                    "global_attn_ms_per_forward": statistics.median(glob),
                    "global_layer_ms": statistics.median(glob) / L}
    log(f"aggregator dense: forward {out['dense']['forward_ms']:.2f} ms, "
        f"global layer {out['dense']['global_layer_ms']:.3f} ms")

    with _ModeEnv("vggt", "vasc"), AttnLaunchEvents(L) as attn_ev:
        install.sparse_aggregator_from_vggt_layerwise(agg, layer_sparsity_ratios=ratios, verbose=False)
        log(f"aggregator vasc: {warmup} warm-up forwards, {steps} timed")
        forwards(warmup, False)
        attn_ev.enabled = True
        total, glob = forwards(steps, True)
        attn_ev.enabled = False
        fwd_ms = total / steps
        out["vasc"] = {"forward_ms": fwd_ms, "frames_per_s": frames / (fwd_ms * 1e-3),
                       "global_attn_ms_per_forward": statistics.median(glob),
                       "global_layer_ms": statistics.median(glob) / L,
                       "frames_per_s_global_layers": frames / (statistics.median(glob) * 1e-3)}
        out["attn_ms_per_launch"] = attn_ev.mean_ms()
        out["attn_launches"] = len(attn_ev.events)
        out["attn_flops_per_launch"] = attn_ev.flops_per_launch()
        counts = [c for _, c, *_ in attn_ev.lists.values()]
        out["mean_listed_blocks_per_row"] = float(torch.stack([c.float().mean() for c in counts]).mean())
    log(f"aggregator vasc: forward {fwd_ms:.2f} ms ({out['vasc']['frames_per_s']:.1f} frames/s), global layer "
        f"{out['vasc']['global_layer_ms']:.3f} ms, attention {out['attn_ms_per_launch']:.3f} ms/launch")
    out["speedup_global_layers_vs_dense"] = out["dense"]["global_layer_ms"] / out["vasc"]["global_layer_ms"]
    del agg, images
    torch.cuda.empty_cache()
    return out


def run_c1(dev, reps: int = 5) -> dict:
    """Config 1 on the GPU: one global layer of 8 frames x 1041 tokens (H=16,
    d=64; N(0,1) plus the per-frame rank-8 component) in vasc mode at
    sparsity 0.75 with a fresh ledger (VGGT official mask), against dense
    attention on the same layer: output differences and the median time of
    ``reps`` calls of each (the vasc call includes pooling, selection with
    the ledger, the V pack and the attention)."""
    from vasc_amd import ops
    from vasc_amd.attention import predict_attention
    from vasc_amd.sparse_wrapper import block_sparse_attn_cuda
    N, P, S, H, D = 8, 1041, 5, 16, 64
    q, k, v = synthetic_layer(N, P, S, H, D, seed=0, device=dev)
    n_patch = q.shape[2]

    def vasc():
        score = predict_attention(q, k[:, :, :n_patch])
        return block_sparse_attn_cuda(q, k, v, score, sparse_ratio=0.75, return_sparsity=True, layer_idx=0,
                                      routing_state={}, num_patch_tokens=n_patch)

    def dense():
        return ops.dense_attn(q, k, ops.pack_v(v))

    times = {}
    with _ModeEnv("vggt", "vasc"):
        for name, fn in (("vasc", vasc), ("dense", dense)):
            fn()
            ms = []
            for _ in range(reps):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                fn()
                b.record()
                torch.cuda.synchronize()
                ms.append(a.elapsed_time(b))
            times[name] = statistics.median(ms)
        out, sparsity = vasc()
    ref = dense().float()
    diff = out.float() - ref
    res = {"vasc_ms": times["vasc"], "dense_ms": times["dense"], "sparsity": float(sparsity),
           "max_abs_vs_dense": float(diff.abs().max()), "mean_abs_vs_dense": float(diff.abs().mean()),
           "rel_l2_vs_dense": float(diff.norm() / ref.norm())}
    log(f"C1: vasc {res['vasc_ms']:.3f} ms, dense {res['dense_ms']:.3f} ms; vasc vs dense max-abs "
        f"{res['max_abs_vs_dense']:.4f}, mean-abs {res['mean_abs_vs_dense']:.5f}, rel L2 {res['rel_l2_vs_dense']:.4f}")
    return res


def kernel_sweeps(layers, ratios, rounds: int = 5) -> dict:
    """Per-launch time of each HBM-bound kernel of the sparse op, launched
    over every layer's inputs back to back between two hipEvents (median of
    ``rounds`` sweeps): the kernels' own duration, without the gaps the
    per-launch events of the step add. Selection runs the chained VASC
    ledger as in the step (its four launches per layer)."""
    from vasc_amd import ops, pipeline
    n_patch = layers[0][0].shape[2]
    pooled = [ops.pool_qkv(q, k[:, :, :n_patch], v[:, :, :n_patch]) for q, k, v in layers]
    probs = [ops.pooled_softmax(pq, pk) for pq, pk, _, _ in pooled]
    plans = [pipeline.LayerPlan.make(n_patch, k.shape[2]) for _, k, _ in layers]
    ledger = pipeline.Ledger()

    def select_all():
        ledger.clear()
        for li, prob in enumerate(probs):
            pipeline.select_layer(prob, pooled[li][3], plans[li], mode="vasc", sparse_ratio=ratios[li],
                                  official_mask=True, ledger=ledger, layer_idx=li)

    sweeps = {
        "pool": lambda: [ops.pool_qkv(q, k[:, :, :n_patch], v[:, :, :n_patch]) for q, k, v in layers],
        "pooled_softmax": lambda: [ops.pooled_softmax(pq, pk) for pq, pk, _, _ in pooled],
        "select": select_all,
        "pack_v": lambda: [ops.pack_v(v) for _, _, v in layers],
    }
    out = {}
    for name, fn in sweeps.items():
        fn()
        out[name] = median_ms(fn, 1, rounds) / len(layers)
    del pooled, probs
    return out


def run_sparse_op(dev, N: int, ratios, steps: int, warmup: int, graph_mode: bool, dense: bool) -> dict:
    """The 24 global layers' sparse op alone (pool + pooled softmax, VASC
    selection with the chained ledger, V pack, block-sparse attention) on
    synthetic Q/K/V resident in HBM: eager steps with hipEvents per kernel,
    then the same step replayed as a HIP graph (checked bit-exact against the
    eager step three times, with eager work in between)."""
    from vasc_amd import ops, pipeline
    P, S, H, D, L = 1041, 5, 16, 64, len(ratios)
    log(f"sparse op: generating {L} layers of synthetic Q/K/V ({N} frames x {P} tokens, H={H})")
    layers = [synthetic_layer(N, P, S, H, D, seed=li, device=dev) for li in range(L)]
    torch.cuda.synchronize()
    ledger = pipeline.Ledger()
    for _ in range(warmup):
        run_step(layers, ratios, ledger, Timer(enabled=False))
    timer = Timer()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    host0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        run_step(layers, ratios, ledger, timer)
    stop.record()
    host_enqueue_ms = (time.perf_counter() - host0) * 1e3 / steps
    torch.cuda.synchronize()
    eager_ms = start.elapsed_time(stop) / steps
    kernel_ms = {k: v / steps for k, v in timer.totals_ms().items()}
    launches = {k: v // steps for k, v in timer.counts().items()}

    keep = []
    run_step(layers, ratios, ledger, Timer(enabled=False), keep)
    n_patch, n_total = N * (P - S), N * P
    attn_flops_step = sum(pipeline.attention_flops((i, c), n_patch, n_total, D) for i, c, _ in keep)
    mins = [attention_min_bytes(i, c, n_patch, n_total, D) for i, c, _ in keep]
    listed_step = sum(int(c.sum().item()) for _, c, _ in keep)
    kernel_bytes = hbm_bytes_per_launch(H, n_patch, n_total, D, listed_step / L)
    eager_out = [o.clone() for _, _, o in keep]
    eager_lists = [(i.clone(), c.clone()) for i, c, _ in keep]
    del keep

    ms_per_step, mode = eager_ms, "eager"
    if graph_mode:
        gkeep = []
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run_step(layers, ratios, ledger, Timer(enabled=False))  # warm the allocator on the side stream
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(graph):
            run_step(layers, ratios, ledger, Timer(enabled=False), gkeep)
        for rep in range(3):  # replays with eager work in between must equal eager bits
            graph.replay()
            torch.cuda.synchronize()
            for (i, c, o), (ei, ec), eo in zip(gkeep, eager_lists, eager_out):
                if not (torch.equal(i, ei) and torch.equal(c, ec) and torch.equal(o.view(torch.int16),
                                                                                 eo.view(torch.int16))):
                    raise RuntimeError(f"graph replay {rep} differs from the eager step")
            run_step(layers[:1], ratios, ledger, Timer(enabled=False))
            torch.cuda.synchronize()
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            graph.replay()
        stop.record()
        torch.cuda.synchronize()
        ms_per_step, mode = start.elapsed_time(stop) / steps, "hip_graph"
        del graph, gkeep

    sweep_ms = kernel_sweeps(layers, ratios)
    attn_ms_launch = kernel_ms["attention"] / launches["attention"]
    achieved = attn_flops_step / L / (attn_ms_launch * 1e-3) / 1e12
    dense_flops_layer = 4.0 * D * H * n_patch * n_total
    out = {
        "description": "24 layers x sparse op (pool+softmax, vasc select + ledger, V pack, block-sparse attention) "
                       "on synthetic N(0,1) + per-frame rank-8 Q/K/V",
        "ms_per_step": ms_per_step, "frames_per_s": N / (ms_per_step * 1e-3), "timing_mode": mode,
        "layer_ms": ms_per_step / L, "eager_ms_per_step": eager_ms, "host_enqueue_ms_per_step": host_enqueue_ms,
        "kernel_ms_per_step": kernel_ms,
        "kernels_hbm": {
            name: {"ms_per_launch": sweep_ms[name], "bytes_per_launch": nbytes,
                   "GB_s": nbytes / (sweep_ms[name] * 1e-3) / 1e9,
                   "frac_of_hbm_peak": nbytes / (sweep_ms[name] * 1e-3) / 1e9 / PEAK_HBM_GBS,
                   "in_step_ms_per_launch": kernel_ms[name] / launches[name]}
            for name, nbytes in kernel_bytes.items()},
        "kernels_hbm_timing": "each kernel over the 24 layers' inputs back to back between two hipEvents "
                              "(median of 5 sweeps); in_step_ms_per_launch: hipEvents around each launch "
                              "inside the eager step (includes the gap to the previous launch)",
        "attention": {"ms_per_launch": attn_ms_launch, "flops_per_launch": attn_flops_step / L,
                      "TFLOP_s": achieved, "frac_of_mfma_peak": achieved / PEAK_BF16_TFLOPS,
                      "min_hbm_bytes_per_launch": statistics.fmean(m[0] for m in mins),
                      "distinct_key_blocks_per_head": statistics.fmean(m[1] for m in mins),
                      "key_blocks_per_head": -(-n_total // 64)},
        "dense_equivalent_TFLOP_s": dense_flops_layer / (ms_per_step / L * 1e-3) / 1e12,
    }
    log(f"sparse op: step {ms_per_step:.3f} ms ({mode}; eager {eager_ms:.3f} ms), attention "
        f"{attn_ms_launch:.3f} ms/layer, {achieved:.1f} TFLOP/s")
    if dense:
        q, k, v = layers[0]
        vt = ops.pack_v(v)
        times = []
        for i in range(4):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            ops.dense_attn(q, k, vt)
            b.record()
            torch.cuda.synchronize()
            if i:
                times.append(a.elapsed_time(b))
        dense_ms = statistics.median(times)
        out["dense_attn_ms"] = dense_ms
        out["dense_attn_TFLOP_s"] = dense_flops_layer / (dense_ms * 1e-3) / 1e12
        out["speedup_vs_dense_attention"] = dense_ms / out["layer_ms"]
        log(f"sparse op: dense attention {dense_ms:.3f} ms/layer, speedup {out['speedup_vs_dense_attention']:.2f}x")
    del layers
    torch.cuda.empty_cache()
    return out


def smooth_images(frames: int, seed: int, dev) -> torch.Tensor:
    """C4's images: rand(1, frames, 3, 28, 37) bilinearly upsampled to 392x518."""
    g = torch.Generator(device=dev).manual_seed(seed)
    low = torch.rand(frames, 3, 28, 37, device=dev, generator=g)
    return torch.nn.functional.interpolate(low, size=(392, 518), mode="bilinear", align_corners=False).unsqueeze(0)


def run_c4(dev, steps: int, warmup: int, tune: bool = True) -> dict:
    """C4: the Pi3-shaped decoder (36 blocks, odd ones global, dim 1024, 16
    heads, 5 register tokens, no camera token, random init bf16) on 64
    frames of seeded smooth noise: dense, then vasc and topk at sparsity 0.75
    with the structural profile (the release default above 0.70), each
    output compared with the dense one."""
    from vasc_amd import install
    from vasc_amd.aggregator import Pi3Decoder
    from vasc_amd.launcher import allocation_settings
    frames = 64
    torch.manual_seed(0)
    with torch.device(dev):
        model = Pi3Decoder(dim=1024, depth=36, num_heads=16, mlp_ratio=4.0)
    model = model.to(torch.bfloat16).eval()
    images = smooth_images(frames, 0, dev)

    def forwards(n):
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.no_grad():
            a.record()
            for _ in range(n):
                y, _ = model(images)
            b.record()
        torch.cuda.synchronize()
        return y, a.elapsed_time(b) / n

    res = {}
    tune_gemms(tune)
    with torch.no_grad():
        forwards(1)  # the warm-up forward tunes the GEMM shapes
    if tune:
        import torch.cuda.tunable as tunable
        tunable.tuning_enable(False)
    with torch.no_grad():
        dense_out, dense_ms = forwards(max(1, steps // 2))
    res["dense"] = {"forward_ms": dense_ms, "frames_per_s": frames / (dense_ms * 1e-3)}
    log(f"C4 dense: forward {dense_ms:.2f} ms")
    ref = dense_out.float()
    for mode in ("vasc", "topk"):
        alloc = allocation_settings("pi3", mode, 0.75, True)
        with _ModeEnv("pi3", mode):
            install.sparse_model_from_pi3(model, sparse_ratio=0.75, layer_sparsity_ratios=alloc["layer_sparsities"],
                                          verbose=False)
            forwards(warmup)
            out, ms = forwards(steps)
        err = (out.float() - ref).abs()
        res[mode] = {"forward_ms": ms, "frames_per_s": frames / (ms * 1e-3),
                     "speedup_vs_dense": dense_ms / ms,
                     "layer_sparsities": alloc["layer_sparsities"],
                     "max_abs_diff_vs_dense": float(err.max()), "mean_abs_diff_vs_dense": float(err.mean()),
                     "dense_output_mean_abs": float(ref.abs().mean())}
        log(f"C4 {mode}: forward {ms:.2f} ms ({res[mode]['frames_per_s']:.1f} frames/s), vs dense max-abs "
            f"{res[mode]['max_abs_diff_vs_dense']:.3e} mean-abs {res[mode]['mean_abs_diff_vs_dense']:.3e}")
        for blk in (model.decoder[i] for i in range(1, len(model.decoder), 2)):  # uninstall: back to dense
            del blk.attn.forward
        model._sparse_routing_state = None
        model._sparse_aux_output_store = None
    del model, images
    torch.cuda.empty_cache()
    return res


def cpu_baseline(frames: int, ratio: float, n_layers: int) -> dict:
    """The reference's CPU-runnable paths restated in torch fp32 on this host's
    cores: C1 (8 frames, 8328 tokens, H=16) dense and topk, one warm-up then
    the median of three; one C2 layer (32 frames) dense and topk, single shot.
    ``value`` scales the C2 topk layer to the 24 global layers' frames/s."""
    from oracle import cpu_baseline as cb
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    out = {}
    c1 = [t.float() for t in synthetic_layer(8, 1041, 5, 16, 64, seed=0, device="cpu")]
    for name, fn in (("topk", lambda: cb.topk_layer(*c1, 0.75)), ("dense", lambda: cb.dense_layer(*c1))):
        times = []
        for i in range(4):
            t0 = time.perf_counter()
            fn()
            if i:
                times.append(time.perf_counter() - t0)
        out[f"c1_{name}_ms"] = statistics.median(times) * 1e3
    log(f"cpu baseline: C1 topk {out['c1_topk_ms']:.1f} ms, dense {out['c1_dense_ms']:.1f} ms on {cores} threads")
    c2 = [t.float() for t in synthetic_layer(frames, 1041, 5, 16, 64, seed=0, device="cpu")]
    t0 = time.perf_counter()
    cb.topk_layer(*c2, ratio)
    topk_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    cb.dense_layer(*c2)
    dense_s = time.perf_counter() - t0
    log(f"cpu baseline: C2 layer topk {topk_s:.2f} s, dense {dense_s:.2f} s")
    out.update({
        "value": frames / (topk_s * n_layers),
        "unit": "frames/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"global attention only: one C2 layer (layer 0, s={ratio:.4f}) of the Top-K path (pooled "
                   f"predictor + top-k + block-gathered attention), torch CPU fp32, single shot, scaled to "
                   f"{n_layers} layers; beside it the same layer dense and C1 (8 frames) dense/topk as the median "
                   f"of 3 after a warm-up"),
        "c2_topk_layer_s": topk_s,
        "c2_dense_layer_s": dense_s,
        "c2_dense_frames_per_s": frames / (dense_s * n_layers),
    })
    return out


def probe_attention(dev) -> int:
    """Untimed, for rocprofv3 --pmc: five launches of the attention kernel at
    the C2 shape (q [1,16,33152,64], k/v [1,16,33312,64] bf16 randn; per query
    block 129 random patch blocks of 518 plus the 3 sink blocks)."""
    from vasc_amd import ops
    H, D, Np, Tk = 16, 64, 33152, 33312
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(1, H, Np, D, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(1, H, Tk, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(1, H, Tk, D, device=dev, generator=g).to(torch.bfloat16)
    qb, kb, kbt = 259, 518, 521
    keys = torch.rand(1, H, qb, kb, device=dev, generator=g)
    pick = torch.topk(keys, 129, dim=-1).indices
    sinks = torch.arange(kb, kbt, device=dev).expand(1, H, qb, kbt - kb)
    index = torch.sort(torch.cat([pick, sinks], -1), -1).values.to(torch.int32).contiguous()
    count = torch.full((1, H, qb), 132, device=dev, dtype=torch.int32)
    vt = ops.pack_v(v)
    for _ in range(5):
        ops.block_sparse_attn(q, k, vt, index, count)
    torch.cuda.synchronize()
    log("attention probe done")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=("c2", "c3", "c4", "c5"), default="c2",
                    help="c2: the metric's configuration (default); c3: 128 frames at s=0.875; c4: the Pi3-shaped "
                         "decoder at 64 frames; c5: per-kernel microbenchmarks at T = 16k/64k/256k")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sparse-op", action="store_true", help="skip the 24-layer sparse-op step (extras)")
    ap.add_argument("--no-gemm-tuning", dest="tune", action="store_false", default=True,
                    help="keep torch's default hipBLASLt GEMM choice (no TunableOp pass in the warm-up)")
    ap.add_argument("--no-graph", dest="graph", action="store_false", default=True,
                    help="time the sparse-op step eagerly only (no HIP graph replay)")
    ap.add_argument("--probe", choices=("attention", "aggregator", "traffic"),
                    help="untimed runs for rocprofv3: five C2 attention launches; three C2 vasc aggregator "
                         "forwards; a 256 MiB copy (counter calibration) then one eager sparse-op step")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the sparse op would shard by head, one head group per GPU). Run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    from vasc_amd import pipeline
    from vasc_amd.launcher import layer_sparsity

    dev = torch.device("cuda:0")
    if args.workload == "c5":
        return run_c5(dev)
    if args.probe == "attention":
        return probe_attention(dev)
    frames, sparsity = {"c2": (32, 0.75), "c3": (128, 0.875), "c4": (64, 0.75)}[args.workload]
    ratios = layer_sparsity("vggt", sparsity, "paper") or [sparsity] * 24
    if args.probe == "aggregator":
        from vasc_amd import install
        agg = build_aggregator(dev)
        g = torch.Generator(device=dev).manual_seed(0)
        images = torch.rand(1, frames, 3, 392, 518, device=dev, generator=g)
        with _ModeEnv("vggt", "vasc"), torch.no_grad():
            install.sparse_aggregator_from_vggt_layerwise(agg, layer_sparsity_ratios=ratios, verbose=False)
            for _ in range(3):
                agg(images)
        torch.cuda.synchronize()
        log("aggregator probe done")
        return 0
    if args.probe == "traffic":
        # a 256 MiB copy (the FETCH_SIZE / WRITE_SIZE scale), then one untimed
        # vasc forward of the headline aggregator
        from vasc_amd import install
        src = torch.empty(128 * 2**20, dtype=torch.bfloat16, device=dev).normal_()
        dst = torch.empty_like(src)
        dst.copy_(src)
        del src, dst
        agg = build_aggregator(dev)
        g = torch.Generator(device=dev).manual_seed(0)
        images = torch.rand(1, frames, 3, 392, 518, device=dev, generator=g)
        with _ModeEnv("vggt", "vasc"), torch.no_grad(), AttnLaunchEvents(len(agg.global_blocks)) as ev:
            install.sparse_aggregator_from_vggt_layerwise(agg, layer_sparsity_ratios=ratios, verbose=False)
            ev.enabled = True
            agg(images)
            ev.enabled = False
        torch.cuda.synchronize()
        mins = [attention_min_bytes_global(*lst) for lst in ev.lists.values()]
        log(f"attention_min_bytes_per_launch: {statistics.fmean(m for m, _ in mins):.0f}")
        log(f"distinct_key_blocks_per_head_patch_queries: {statistics.fmean(b for _, b in mins):.2f}")
        log("traffic probe done")
        return 0

    if args.workload == "c4":
        c4 = run_c4(dev, args.steps, args.warmup, tune=args.tune)
        v = c4["vasc"]
        result = {
            "metric": "Pi3-shaped decoder forward, vasc @75% sparsity, 64 frames; frames/s",
            "value": v["frames_per_s"], "unit": "frames/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": v["forward_ms"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic: seeded smooth noise (28x37 uniform noise bilinearly upsampled to 392x518)",
            "config": {"workload": "C4 Pi3-shaped decoder forward (36 blocks, 18 global), vasc and topk vs dense",
                       "frames": frames, "tokens": frames * 1041, "heads": 16, "head_dim": 64, "dim": 1024,
                       "sparsity": sparsity, "structural_allocation": True,
                       "block_gemms": "hipBLASLt via torch" + (", TunableOp-tuned in the warm-up" if args.tune else "")},
            "c4": c4,
        }
        print(json.dumps(result), flush=True)
        return 0

    N, P, S, H, D, L = frames, 1041, 5, 16, 64, 24
    agg = run_aggregator(dev, N, ratios, args.steps, args.warmup, dense_reps=3 if args.workload == "c2" else 1,
                         tune=args.tune)
    v = agg["vasc"]
    achieved = agg["attn_flops_per_launch"] / (agg["attn_ms_per_launch"] * 1e-3) / 1e12
    result = {
        "metric": METRIC if args.workload == "c2" else
        f"sparse global-attn layer ms + eff. TFLOP/s @{sparsity:g} sparsity, {N} frames; frames/s",
        "value": v["frames_per_s"],
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": v["forward_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic: random-init bf16 weights, seeded uniform-noise images [1,{N},3,392,518]",
        "config": {
            "workload": f"{args.workload.upper()} VGGT-shaped aggregator forward (24 frame + 24 global blocks, "
                        f"dim 1024, 16 heads, MLP 4096) with the vasc sparse global attention",
            "frames": N, "tokens": N * P, "patch_tokens": N * (P - S), "heads": H, "head_dim": D,
            "global_layers": L, "mode": "vasc", "sparsity": sparsity, "structural_allocation": True,
            "block_gemms": "hipBLASLt via torch" + (", TunableOp-tuned in the warm-up" if args.tune else ""),
        },
        "global_layer_ms": v["global_layer_ms"],
        "frames_per_s_global_layers": v["frames_per_s_global_layers"],
        "speedup_global_layer_vs_dense": agg["speedup_global_layers_vs_dense"],
        "aggregator": agg,
        "roofline": {
            "kernel": "bsattn_fwd_kernel (vasc_global_attn_tokens_fwd: patch queries over their lists + special queries, results on the frame-major token rows)",
            "bound": "mfma",
            "achieved": achieved,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / PEAK_BF16_TFLOPS,
            "traffic": traffic_bytes() if args.workload == "c2" else None,
            "traffic_source": TRAFFIC_SUMMARY if args.workload == "c2" else None,
            "flops_per_launch": agg["attn_flops_per_launch"],
            "ms_per_launch": agg["attn_ms_per_launch"],
            "launches_timed": agg["attn_launches"],
        },
    }
    if not args.no_sparse_op:
        result["sparse_op"] = run_sparse_op(dev, N, ratios, args.steps, args.warmup, args.graph, dense=True)
    if args.workload == "c2":
        result["c1"] = run_c1(dev)
    if not args.no_cpu_baseline and args.workload == "c2":
        result["cpu_baseline"] = cpu_baseline(N, ratios[0], L)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
