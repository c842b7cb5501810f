"""Benchmark of the MI355X Qwen3-MoE FP8 expert layer (one GPU).

One step = one MoE block forward (router + FP8 experts) over one batch of synthetic
tokens already resident in HBM.  The headline line is the Qwen3-30B-A3B-shaped layer
(hidden 2048, 128 experts, top-8, moe_intermediate 768, 128x128 block scales) at a
decode batch of 64 tokens.  The sweep adds the other decode batches,
the 4096-token Zipf-skewed prefill chunk (config 3) and the Qwen3-235B-A22B shape
(hidden 4096, moe_intermediate 1536) at decode 64 and prefill 2048 (config 4).

Weights are rotated over enough copies that one step's weights never sit in the 256 MB
last-level cache from an earlier step; inputs rotate too, so routing changes every step.

The decode-step entry (config 5) runs a 48-layer Qwen3-30B-A3B-shaped decode step at batch 128:
per layer RMSNorm, bf16 q/k/v projections, q/k norm, rotary, KV append, paged GQA attention over
contexts uniform in [512, 8192] (page size 16), o_proj, RMSNorm and the FP8 MoE block, all layers
replayed as one HIP graph; it reports decode tokens/s and the per-layer MoE and attention shares.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--tokens 64] [--zipf] [--no-sweep]
                       [--no-cpu] [--no-decode-step] [--decode-step-only] [--copy-probe] [--library-probe] [--shape 30b|235b]
  --zipf        apply the calibrated Zipf(s=1.1) router bias to the headline batch (config 3)
  --copy-probe  first run a plain 256 MiB device copy three times: the reference kernel whose
                FETCH_SIZE / WRITE_SIZE counters calibrate the traffic measurement
  --library-probe  time the vendor's dense FP8 / bf16 GEMMs on the expert GEMM shapes (a ceiling
                reference for the grouped kernels) and exit
  --shape 235b  the headline line on the Qwen3-235B-A22B layer instead (with --no-sweep, for profiling)
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from dataclasses import dataclass

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = "MoE layer µs + % roofline (HBM GB/s / FP8 MFMA), Qwen3-30B-A3B shape, bs 1–4096"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
LLC_BYTES = 256 * 2 ** 20
K_TOP = 8
N_SLOTS = 9  # kernel timing slots of the library (include/moe_mi355x.h)


@dataclass(frozen=True)
class Shape:
    name: str
    H: int
    I: int
    E: int = 128

    def gate_up_expert_bytes(self):
        """W13 + its scales of one expert: 3,146,496 B for the 30B shape."""
        return 2 * self.I * self.H + 4 * (2 * self.I // 128) * (self.H // 128)

    def expert_bytes(self):
        """W13 + W2 + scales of one expert: 4,719,744 B for the 30B shape."""
        return self.gate_up_expert_bytes() + self.H * self.I + 4 * (self.H // 128) * (self.I // 128)

    def gate_up_bytes(self, n_active, T):
        """Algorithmic HBM bytes of one gate_up launch: the active experts' W13 + scales,
        the fp8 activations and their scales read, the intermediate written: bf16 h, which the
        16-row down GEMM quantises as it loads it where its LDS rows hold I (I <= 1024); else up
        to 2 pairs per expert (S <= 2 E) the launch quantises it itself (e4m3 codes + scales, and
        its bf16 h round trip between the launch's workgroups is counted too).  On the 128-row
        prefill path the launch writes the e4m3 codes of h and their scales."""
        S = T * K_TOP
        if self.prefill_path(T):  # the 128-row kernel writes the e4m3 codes of h and their scales
            out = S * self.I + 4 * S * (self.I // 128)
            return n_active * self.gate_up_expert_bytes() + T * self.H + 4 * T * (self.H // 128) + out
        out = 2 * S * self.I
        down_quantises = S <= 8 * self.E and self.I <= 1024 and not (self.I == 1024 and S > 16)
        if S <= 2 * self.E and not down_quantises:
            out += 2 * S * self.I + S * self.I + 4 * S * (self.I // 128)
        return n_active * self.gate_up_expert_bytes() + T * self.H + 4 * T * (self.H // 128) + out

    def gate_up_flops(self, T):
        return 2.0 * T * K_TOP * (2 * self.I) * self.H

    def layer_bytes(self, n_active, T):
        return n_active * self.expert_bytes() + 2 * self.E * self.H + 4 * T * self.H

    def layer_flops(self, T):
        return T * K_TOP * (2.0 * self.H * 2 * self.I + 2.0 * self.I * self.H) + 2.0 * T * self.H * self.E

    def expected_active(self, T):
        return self.E * (1.0 - (1.0 - K_TOP / self.E) ** T)

    def bf16_gate_up_bytes(self, n_active, T):
        """bf16 experts: the active experts' W13, x read, bf16 h written."""
        return n_active * 2 * (2 * self.I * self.H) + 2 * T * self.H + 2 * T * K_TOP * self.I

    def bf16_layer_bytes(self, n_active, T):
        return n_active * 2 * 3 * self.I * self.H + 2 * self.E * self.H + 4 * T * self.H

    def prefill_path(self, T):
        """True where the library picks the 128-row MFMA-tiled (compute-bound) GEMMs: beyond 8
        pairs per expert, for a hidden size in 256-column tiles and both GEMMs >= 4 K blocks."""
        return T * K_TOP > 8 * self.E and self.H % 256 == 0 and self.H >= 512 and self.I >= 512


S30B = Shape("qwen3-30b-a3b", 2048, 768)
S235B = Shape("qwen3-235b-a22b", 4096, 1536)

# HBM bytes per gate_up launch measured with two rocprofv3 --pmc runs of this script on the build of
# commit a71d4f3 (FETCH_SIZE x 2.00 + WRITE_SIZE x 1.00, KiB; the factors calibrated on a 256 MiB copy);
# commands and per-dispatch figures in profiles/grouped_gemm_hbm_traffic.md:
#   decode 64:            FETCH 195,261 / WRITE 768 KiB
#   prefill 4096, Zipf:   FETCH 292,772 / WRITE 25,458 KiB
_TRAFFIC_SRC = "profiles/grouped_gemm_hbm_traffic.md (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, build of a71d4f3)"
MEASURED_GATE_UP_TRAFFIC = {
    ("qwen3-30b-a3b", 64): {"bytes": 195261 * 1024 * 2 + 768 * 1024, "source": _TRAFFIC_SRC},
    ("qwen3-30b-a3b", 4096): {"bytes": 292772 * 1024 * 2 + 25458 * 1024, "source": _TRAFFIC_SRC},
}


class Layer:
    """Router + FP8 experts of one shape, with `n_copies` distinct copies of the experts."""

    def __init__(self, pkg, torch, dev, shape, n_copies):
        self.shape = shape
        E, H, I = shape.E, shape.H, shape.I
        g = torch.Generator(device=dev).manual_seed(0)
        self.wr = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        w13 = (torch.randn((E, 2 * I, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        q13, s13 = pkg.quantize_weight_fp8(w13)
        del w13
        w2 = (torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        q2, s2 = pkg.quantize_weight_fp8(w2)
        del w2
        self.copies = [(q13, s13, q2, s2)] + [tuple(t.clone() for t in (q13, s13, q2, s2))
                                             for _ in range(n_copies - 1)]

    def n_rot(self, T):
        per_step = self.shape.layer_bytes(self.shape.expected_active(T), T)
        return max(2, min(len(self.copies), math.ceil(2 * LLC_BYTES / max(1.0, per_step))))


class Bf16Layer:
    """Router + bf16 experts of one shape (the reference's default checkpoint dtype, run on the
    library's bf16 path), with `n_copies` distinct copies of the experts."""

    def __init__(self, torch, dev, shape, n_copies, wr):
        self.shape = shape
        self.wr = wr
        g = torch.Generator(device=dev).manual_seed(7)
        self.copies = []
        for _ in range(n_copies):
            w13 = (torch.randn((shape.E, 2 * shape.I, shape.H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
            w2 = (torch.randn((shape.E, shape.H, shape.I), generator=g, device=dev) * 0.02).to(torch.bfloat16)
            self.copies.append((w13, w2))

    def n_rot(self, T):
        return len(self.copies)


def make_inputs(torch, dev, shape, T, n, zipf_beta=None):
    g = torch.Generator(device=dev).manual_seed(1000 + T)
    xs = [torch.randn((T, shape.H), generator=g, device=dev).to(torch.bfloat16) for _ in range(n)]
    if zipf_beta is not None:
        for x in xs:  # hidden dim 0 carries a constant 1, router column 0 the Zipf bias
            x[:, 0] = 1.0
    return xs


def zipf_router(torch, wr, beta):
    import numpy as np

    E = wr.shape[0]
    r = np.random.default_rng(0).permutation(E) + 1
    b = torch.tensor(beta * (-1.1 * np.log(r)), dtype=torch.float32, device=wr.device)
    w = wr.clone()
    w[:, 0] = b.to(torch.bfloat16)
    return w


def calibrate_zipf(pkg, torch, dev, layer, T=4096):
    """Bisect beta so that the 10 most loaded experts take 50% of the T*k assignments."""
    x = make_inputs(torch, dev, layer.shape, T, 1, zipf_beta=0.0)[0]
    lo, hi = 0.0, 8.0
    share = 0.0
    for _ in range(24):
        mid = 0.5 * (lo + hi)
        _, _, ids = pkg.route(x, zipf_router(torch, layer.wr, mid), K_TOP)
        cnt = torch.bincount(ids.reshape(-1), minlength=layer.shape.E).sort(descending=True).values
        share = float(cnt[:10].sum()) / (T * K_TOP)
        if share < 0.5:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi), share


def run_config(pkg, torch, layer, T, steps, warmup, router, xs):
    """Times `steps` block forwards, then runs them again under the library's per-kernel
    HIP events.  Returns (ms per step, per-slot average ms, mean active experts, copies).
    A Bf16Layer runs the bf16-expert block, a Layer the FP8 one."""
    lib = pkg._lib.load()
    n_rot = layer.n_rot(T)
    block = pkg.moe_block_bf16 if isinstance(layer, Bf16Layer) else pkg.moe_block_fp8

    def step(i, routing=False):
        return block(xs[i % len(xs)], router, K_TOP, *layer.copies[i % n_rot], return_routing=routing)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for i in range(steps):
        step(i)
    en.record()
    torch.cuda.synchronize()
    ms = st.elapsed_time(en) / steps

    lib.moe_mi355x_profile_enable(1)
    ids_seen = []
    for i in range(steps):
        _, (_, _, ids) = step(i, routing=True)
        ids_seen.append(ids)
    torch.cuda.synchronize()
    slots = {}
    for slot in range(N_SLOTS):
        if not lib.moe_mi355x_profile_slot_name(slot):
            continue
        n, tot = ctypes.c_int(0), ctypes.c_double(0.0)
        pkg._lib.check(lib.moe_mi355x_profile_read(slot, ctypes.byref(n), ctypes.byref(tot)), "profile_read")
        if n.value:
            slots[lib.moe_mi355x_profile_slot_name(slot).decode()] = tot.value / steps
    lib.moe_mi355x_profile_enable(0)
    active = [int(torch.unique(ids).numel()) for ids in ids_seen]
    return ms, slots, sum(active) / len(active), n_rot


def graph_step_ms(pkg, torch, layer, T, steps, router, xs):
    """Per-step time when the steps replay a captured HIP graph: one graph holds a whole weight
    rotation (one block call per weight copy, as a decode step's graph holds all its layers), so
    the figure is the GPU's time per layer without host launch cost per call."""
    n_rot = layer.n_rot(T)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for j in range(n_rot):
            pkg.moe_block_fp8(xs[j % len(xs)], router, K_TOP, *layer.copies[j])
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for j in range(n_rot):
            pkg.moe_block_fp8(xs[j % len(xs)], router, K_TOP, *layer.copies[j])
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, math.ceil(steps / n_rot))
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(reps):
        g.replay()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) / (reps * n_rot)


RIDGE_FLOP_PER_BYTE = FP8_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)  # 625 flop/B


def roofline_for(shape, T, slots, n_active):
    """Roofline of the dominant kernel, gate_up.  The bound follows its arithmetic intensity
    (algorithmic flops over algorithmic HBM bytes of the measured active experts) against the
    ridge of the FP8 peak and HBM (625 flop/B): below it the launch is HBM-bound and `frac` is
    the HBM fraction, above it MFMA-bound and `frac` the FP8 fraction.  Both fractions are
    reported (`hbm_frac`, `mfma_frac`): the prefill chunks sit just below the ridge (4096 tokens
    ~470 flop/B), where both roofs are close."""
    dur_ms = slots["gemm_gate_up"]
    traffic = MEASURED_GATE_UP_TRAFFIC.get((shape.name, T))
    flops = shape.gate_up_flops(T)
    byts = shape.gate_up_bytes(n_active, T)
    gbs = byts / (dur_ms * 1e-3) / 1e9
    tflops = flops / dur_ms / 1e9
    intensity = flops / byts
    out = {"kernel": "gemm_gate_up", "intensity_flop_per_byte": round(intensity, 1),
           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "mfma_frac": round(tflops / FP8_PEAK_TFLOPS, 4),
           "traffic": traffic["bytes"] if traffic else None,
           "traffic_source": traffic["source"] if traffic else None,
           "algorithmic_bytes": int(byts), "algorithmic_flop": flops, "avg_us": round(dur_ms * 1e3, 2)}
    if intensity >= RIDGE_FLOP_PER_BYTE:
        out.update(bound="mfma", achieved=round(tflops, 1), peak=FP8_PEAK_TFLOPS, unit="TFLOP/s",
                   frac=out["mfma_frac"])
    else:
        out.update(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s", frac=out["hbm_frac"])
    return out


def bf16_sweep_entry(pkg, torch, dev, layer, T, steps, zipf=None):
    """The bf16-expert block (the reference's default bf16 checkpoint, no FP8 requantisation):
    decode batches are HBM-bound, the 128-row prefill tiles bf16-MFMA-bound."""
    shape = layer.shape
    beta = share = None
    router = layer.wr
    if zipf is not None:
        beta, share = zipf
        router = zipf_router(torch, layer.wr, beta)
    xs = make_inputs(torch, dev, shape, T, 4, zipf_beta=beta)
    ms, slots, act, _ = run_config(pkg, torch, layer, T, steps, 20, router, xs)
    dur_ms = slots["gemm_gate_up"]
    entry = {"shape": shape.name, "experts_dtype": "bf16", "tokens": T, "us_per_layer": round(ms * 1e3, 2),
             "tokens_per_s": round(T / (ms * 1e-3), 1), "mean_active_experts": round(act, 2),
             "kernels_us": {k: round(v * 1e3, 2) for k, v in slots.items()}}
    # bound by arithmetic intensity against the bf16 ridge (2.5 PFLOP/s over 8 TB/s = 312.5 flop/B)
    flops = shape.gate_up_flops(T)
    byts = shape.bf16_gate_up_bytes(act, T)
    gbs = byts / (dur_ms * 1e-3) / 1e9
    tflops = flops / dur_ms / 1e9
    rf = {"kernel": "gemm_gate_up", "intensity_flop_per_byte": round(flops / byts, 1),
          "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
          "traffic": None, "algorithmic_bytes": int(byts), "algorithmic_flop": flops, "avg_us": round(dur_ms * 1e3, 2)}
    if flops / byts >= BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9):
        rf.update(bound="mfma", achieved=round(tflops, 1), peak=BF16_PEAK_TFLOPS, unit="TFLOP/s", frac=rf["mfma_frac"])
    else:
        rf.update(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s", frac=rf["hbm_frac"])
    entry["roofline"] = rf
    entry["layer_tflops"] = round(shape.layer_flops(T) / (ms * 1e-3) / 1e12, 1)
    entry["layer_bf16_peak_frac"] = round(entry["layer_tflops"] / BF16_PEAK_TFLOPS, 4)
    entry["layer_hbm_frac"] = round(shape.bf16_layer_bytes(act, T) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    if zipf is not None:
        entry["routing"] = f"zipf s=1.1 bias, beta={beta:.3f}, top-10 share={share:.3f}"
    print(json.dumps({"sweep_progress": entry}), file=sys.stderr, flush=True)
    return entry


def sweep_entry(pkg, torch, dev, layer, T, steps, zipf=None):
    shape = layer.shape
    beta = share = None
    router = layer.wr
    if zipf is not None:
        beta, share = zipf
        router = zipf_router(torch, layer.wr, beta)
    xs = make_inputs(torch, dev, shape, T, 4, zipf_beta=beta)
    ms, slots, act, _ = run_config(pkg, torch, layer, T, steps, 20, router, xs)
    entry = {"shape": shape.name, "experts_dtype": "fp8", "tokens": T, "us_per_layer": round(ms * 1e3, 2),
             "tokens_per_s": round(T / (ms * 1e-3), 1),
             "us_per_layer_graph": round(graph_step_ms(pkg, torch, layer, T, steps, router, xs) * 1e3, 2),
             "mean_active_experts": round(act, 2), "roofline": roofline_for(shape, T, slots, act),
             "kernels_us": {k: round(v * 1e3, 2) for k, v in slots.items()}}
    if zipf is not None:
        entry["routing"] = f"zipf s=1.1 bias, beta={beta:.3f}, top-10 share={share:.3f}"
    entry["layer_tflops"] = round(shape.layer_flops(T) / (ms * 1e-3) / 1e12, 1)
    entry["layer_mfma_frac"] = round(entry["layer_tflops"] / FP8_PEAK_TFLOPS, 4)
    entry["layer_hbm_frac"] = round(shape.layer_bytes(act, T) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    entry["layer_bound"] = "mfma" if shape.layer_flops(T) / shape.layer_bytes(act, T) >= RIDGE_FLOP_PER_BYTE else "hbm"
    print(json.dumps({"sweep_progress": entry}), file=sys.stderr, flush=True)
    return entry


def ep_share_entry(pkg, torch, dev, shape=None, e_local=16, steps=40):
    """One GPU's share of an 8-way expert-parallel layer: E/8 local experts at the real H / I, fed
    the rows the dispatch all-to-all would deliver (each of 8 GPUs' T tokens sends its k slots to
    the slots' owners, so a GPU receives T k rows on average, one expert each: the experts entry
    point with k = 1, ids uniform over the local experts).  The exchanges themselves are not
    timed (one GPU).  Bytes: the local experts' weights and scales plus bf16 rows in and out."""
    shape = shape or S30B
    E, H, I = e_local, shape.H, shape.I
    g = torch.Generator(device=dev).manual_seed(5)
    copies = []
    for _ in range(4):  # 4 x 75 MB rotated: more than the 256 MB last-level cache
        w13 = (torch.randn((E, 2 * I, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        q13, s13 = pkg.quantize_weight_fp8(w13)
        del w13
        w2 = (torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        q2, s2 = pkg.quantize_weight_fp8(w2)
        del w2
        copies.append((q13, s13, q2, s2))
    per_expert = shape.expert_bytes()
    out = []
    for T in (1, 8, 64, 128):
        R = T * K_TOP
        x = torch.randn((R, H), generator=g, device=dev).to(torch.bfloat16)
        ids = torch.randint(0, E, (R, 1), generator=g, device=dev, dtype=torch.int64)
        wts = torch.ones((R, 1), device=dev, dtype=torch.bfloat16)
        active = int(torch.unique(ids).numel())
        for i in range(5):
            pkg.experts_fp8(x, ids, wts, *copies[i % 4])
        torch.cuda.synchronize()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        for i in range(steps):
            pkg.experts_fp8(x, ids, wts, *copies[i % 4])
        en.record()
        torch.cuda.synchronize()
        us = st.elapsed_time(en) / steps * 1e3
        nbytes = active * per_expert + 4 * R * H
        out.append({"tokens_per_gpu": T, "rows_received": R, "local_experts": E, "active": active,
                    "us": round(us, 2), "bytes": nbytes, "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    del copies
    torch.cuda.empty_cache()
    return {"workload": f"{shape.name} experts, one GPU's share of 8-way expert parallelism "
                        f"({e_local} local experts, T*k received rows with k = 1)", "points": out}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, layer, router, x, warmup=3, runs=10):
    """The reference's PyTorch CPU path (oracle/torch_ref.py: transformers' router and
    grouped_mm experts forward restated op for op, FP8 weights dequantised once to fp32, dynamic
    activation quantisation), timed on this host's cores on the headline workload: `warmup`
    untimed block forwards, then the median of `runs`."""
    from oracle import torch_ref

    # the box grants this job a CPU share (OMP_NUM_THREADS) that can be far below os.cpu_count()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        q13, s13, q2, s2 = (t.cpu() for t in layer.copies[0])
        w13f = torch_ref.dequantize_weight(q13, s13)
        w2f = torch_ref.dequantize_weight(q2, s2)
        xc, wrc = x.cpu(), router.cpu()
        T = xc.shape[0]
        times = []
        with torch.no_grad():
            for i in range(warmup + runs):
                t0 = time.perf_counter()
                torch_ref.block_fp8_dequant(xc, wrc, K_TOP, w13f, w2f)
                if i >= warmup:
                    times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev_threads)
    med = sorted(times)[len(times) // 2]
    return {"value": round(T / med, 2), "unit": "tokens/s", "us_per_layer": round(med * 1e6, 1),
            "cores": threads, "os_cpu_count": os.cpu_count(), "cpu_model": _cpu_model(), "kind": "port",
            "impl": "torch CPU (the reference's DEVICE=cpu path: transformers router + grouped_mm experts "
                    "forward restated in torch, oracle/torch_ref.py)",
            "sample": f"the {T}-token headline batch: {warmup} warm-up block forwards, median of {runs} "
                      f"(router, sort, histc, cumsum, fp32 grouped_mm on FP8 weights dequantised once, "
                      f"dynamic activation quantisation, combine), torch.set_num_threads({threads})"}


def decode_step_entry(pkg, torch, dev, steps=10, n_layers=48, batch=128, seed=0):
    """a 48-layer Qwen3-30B-A3B-shaped decode step at batch 128, random-init
    FP8 experts and bf16 dense weights, bf16 GQA paged attention (32 q / 4 kv heads, head_dim 128,
    page 16) over context lengths uniform in [512, 8192] (the new token included).  Every
    replay re-appends the same token, so each step does the same work."""
    import numpy as np

    from inference_server_amd import decode as dec

    cfg = dec.DecoderConfig()
    rng = np.random.default_rng(seed)
    lens = rng.integers(512, 8193, size=batch).astype(np.int32)
    pages_per_seq = (lens + dec.PAGE_SIZE - 1) // dec.PAGE_SIZE
    n_pages = int(pages_per_seq.sum())
    max_pages = int(pages_per_seq.max())
    order = torch.randperm(n_pages, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    tables = torch.zeros((batch, max_pages), dtype=torch.int32)
    used = 0
    for b in range(batch):
        tables[b, : pages_per_seq[b]] = order[used: used + pages_per_seq[b]]
        used += int(pages_per_seq[b])
    tables = tables.to(dev)
    ctx = torch.from_numpy(lens).to(dev)
    gen = torch.Generator(device=dev).manual_seed(seed)
    layers = [dec.DecoderLayerWeights.random(cfg, dev, gen) for _ in range(n_layers)]
    cache = dec.PagedKVCache(n_layers, n_pages, cfg.kv_heads, dev)
    for t in cache.k + cache.v:
        t.normal_(generator=gen)
    h = torch.randn((batch, cfg.hidden), generator=gen, device=dev).to(torch.bfloat16)
    model = dec.DecodeModel(cfg, layers, cache)

    def timed(graph):
        for _ in range(2):
            graph.replay()
        torch.cuda.synchronize()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        for _ in range(steps):
            graph.replay()
        en.record()
        torch.cuda.synchronize()
        return st.elapsed_time(en) / steps

    res = {}
    with torch.no_grad():
        for name, kw in (("full", {}), ("attention_only", {"moe": False}), ("moe_only", {"attention": False})):
            graph, statics, out = model.capture(h, ctx - 1, ctx, tables, **kw)
            res[name] = timed(graph)
            assert torch.isfinite(out.float()).all(), f"non-finite hidden states ({name})"
            del graph, statics, out
        # the attention kernel alone, every layer's cache once (HIP events on the launch stream)
        q = torch.randn((batch, cfg.heads, cfg.head_dim), generator=gen, device=dev).to(torch.bfloat16)
        for i in range(2):
            pkg.paged_attention_decode(q, cache.k[i], cache.v[i], tables, ctx, cfg.head_dim ** -0.5)
        torch.cuda.synchronize()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        for i in range(n_layers):
            pkg.paged_attention_decode(q, cache.k[i], cache.v[i], tables, ctx, cfg.head_dim ** -0.5)
        en.record()
        torch.cuda.synchronize()
        attn_kernel_ms = st.elapsed_time(en) / n_layers
    kv_bytes = int(lens.sum()) * cfg.kv_heads * cfg.head_dim * 2 * 2  # K and V, bf16
    ms = res["full"]
    entry = {
        "workload": f"qwen3-30b-a3b {n_layers}-layer decode step, batch {batch}, bf16 GQA paged attention "
                    f"(32 q / 4 kv heads, head_dim 128, page 16), contexts U[512, 8192] (mean {lens.mean():.0f}), "
                    "fp8 experts; all layers in one HIP graph",
        "data": "synthetic (random-init weights, random KV cache)",
        "ms_per_step": round(ms, 4),
        "tokens_per_s": round(batch / (ms * 1e-3), 1),
        "us_per_layer": round(ms * 1e3 / n_layers, 2),
        "attention_layers_us_per_layer": round(res["attention_only"] * 1e3 / n_layers, 2),
        "moe_layers_us_per_layer": round(res["moe_only"] * 1e3 / n_layers, 2),
        "moe_share": round(res["moe_only"] / ms, 4),
        "attention_kernel": {"us": round(attn_kernel_ms * 1e3, 2), "kv_bytes": kv_bytes,
                             "achieved_gbs": round(kv_bytes / (attn_kernel_ms * 1e-3) / 1e9, 1),
                             "hbm_frac": round(kv_bytes / (attn_kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
    }
    del model, layers, cache
    torch.cuda.empty_cache()
    print(json.dumps({"decode_step_progress": entry}), file=sys.stderr, flush=True)
    return entry


def library_probe(torch, dev, reps=50):
    """The library's dense GEMMs on the expert GEMMs' shapes: ``torch._scaled_mm`` (FP8 e4m3 x e4m3,
    one fp32 scale per tensor, bf16 out) and the bf16 matmul, both hipBLASLt on this build, with
    HIP events on torch's current stream (where the library launches).  Rows are token-expert
    pairs: all 32768 pairs of the 4096-token prefill chunk as one dense GEMM (no grouping, no block
    scales, no gather, no fused SiLU or quantisation: an upper bound for what a grouped kernel of
    the same shape can reach), one hot expert's rows (3222 under the Zipf routing), one cold
    expert's (139), and the library's best case 8192^3."""
    shapes = [("gate_up, all pairs", 32768, 1536, 2048), ("down, all pairs", 32768, 2048, 768),
              ("gate_up, hot expert", 3222, 1536, 2048), ("gate_up, cold expert", 139, 1536, 2048),
              ("square", 8192, 8192, 8192)]
    out = []
    for name, M, N, K in shapes:
        a = torch.randn((M, K), device=dev).to(torch.float8_e4m3fn)
        b = torch.randn((N, K), device=dev).to(torch.float8_e4m3fn)
        one = torch.ones((), device=dev)
        ab, bb = torch.randn((M, K), device=dev, dtype=torch.bfloat16), torch.randn((N, K), device=dev, dtype=torch.bfloat16)
        fns = {"fp8": (lambda: torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16), 5000.0),
               "bf16": (lambda: ab @ bb.t(), 2500.0)}
        entry = {"gemm": name, "M": M, "N": N, "K": K}
        for dt, (fn, peak) in fns.items():
            for _ in range(5):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
            entry[dt] = {"us": round(us, 2), "tflops": round(tf, 1), "peak_frac": round(tf / peak, 4)}
        out.append(entry)
        del a, b, ab, bb
    # the floor of one dependent launch: back-to-back tiny elementwise kernels on one stream
    t = torch.zeros(64, device=dev)
    for _ in range(10):
        t.add_(1.0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(1000):
        t.add_(1.0)
    e1.record()
    torch.cuda.synchronize()
    out.append({"gemm": "none: one tiny elementwise kernel per launch, 1000 back to back",
                "us_per_launch": round(e0.elapsed_time(e1) * 1e3 / 1000, 2)})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--zipf", action="store_true")
    ap.add_argument("--copy-probe", action="store_true")
    ap.add_argument("--library-probe", action="store_true",
                    help="time the vendor GEMMs (hipBLASLt through torch) on dense shapes of the expert "
                         "GEMMs, as a ceiling reference for the grouped kernels; prints one JSON object")
    ap.add_argument("--no-decode-step", action="store_true", help="skip the 48-layer decode step (config 5)")
    ap.add_argument("--decode-step-only", action="store_true", help="run only the 48-layer decode step")
    ap.add_argument("--shape", choices=["30b", "235b"], default="30b",
                    help="layer of the headline line: Qwen3-30B-A3B (default) or Qwen3-235B-A22B")
    ap.add_argument("--experts-dtype", choices=["fp8", "bf16"], default="fp8",
                    help="bf16: time only the bf16-expert block of the 30B layer at --tokens (one JSON "
                         "entry, for profiling); the headline line is always the FP8 block")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (expert-parallel sharding "
              "is a design note); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    pkg._lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe:
        src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.decode_step_only:
        print(json.dumps({"decode_step": decode_step_entry(pkg, torch, dev)}), flush=True)
        return
    if args.library_probe:
        print(json.dumps({"library_probe": library_probe(torch, dev)}), flush=True)
        return
    if args.experts_dtype == "bf16":
        g = torch.Generator(device=dev).manual_seed(0)
        wr = (torch.randn((S30B.E, S30B.H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        b16 = Bf16Layer(torch, dev, S30B, 2, wr)
        zipf = calibrate_zipf(pkg, torch, dev, b16, T=args.tokens) if args.zipf else None
        print(json.dumps({"bf16_block": bf16_sweep_entry(pkg, torch, dev, b16, args.tokens, args.steps, zipf=zipf)}),
              flush=True)
        return
    layer = Layer(pkg, torch, dev, S30B, n_copies=16) if args.shape == "30b" else Layer(pkg, torch, dev, S235B, n_copies=2)
    shape = layer.shape

    T = args.tokens
    beta = share = None
    router = layer.wr
    if args.zipf:
        beta, share = calibrate_zipf(pkg, torch, dev, layer, T=T)
        router = zipf_router(torch, layer.wr, beta)
    xs = make_inputs(torch, dev, shape, T, 8, zipf_beta=beta)
    ms, slots, n_active, n_rot = run_config(pkg, torch, layer, T, args.steps, args.warmup, router, xs)
    line = {
        "metric": METRIC,
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_layer": round(ms * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic",
        "config": {"workload": f"{shape.name} moe layer, fp8 128x128 block scales, "
                               f"{'prefill chunk' if shape.prefill_path(T) else 'decode batch'} {T}",
                   "tokens": T, "hidden": shape.H, "experts": shape.E, "top_k": K_TOP,
                   "moe_intermediate": shape.I,
                   "routing": (f"zipf s=1.1 router bias, beta={beta:.3f}, top-10 share={share:.3f}" if args.zipf
                               else "router-driven (x~N(0,1), W_r~N(0,0.02): uniform in distribution)"),
                   "weight_copies_rotated": n_rot, "mean_active_experts": round(n_active, 2)},
        "roofline": roofline_for(shape, T, slots, n_active),
        "kernels_us": {k: round(v * 1e3, 2) for k, v in slots.items()},
        "layer_hbm_frac": round(shape.layer_bytes(n_active, T) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "us_per_layer_graph": round(graph_step_ms(pkg, torch, layer, T, args.steps, router, xs) * 1e3, 2),
    }
    if not args.no_sweep:
        sweep = []
        zipf = calibrate_zipf(pkg, torch, dev, layer)
        for Ts in (1, 8, 32, 64, 128, 256, 4096):
            sweep.append(sweep_entry(pkg, torch, dev, layer, Ts, 100 if Ts < 4096 else 20,
                                     zipf=zipf if Ts == 4096 else None))
        big = Layer(pkg, torch, dev, S235B, n_copies=2)
        for Ts in (64, 2048):
            sweep.append(sweep_entry(pkg, torch, dev, big, Ts, 100 if Ts < 2048 else 20))
        del big
        torch.cuda.empty_cache()
        b16 = Bf16Layer(torch, dev, S30B, 2, layer.wr)
        for Ts in (1, 64, 4096):
            sweep.append(bf16_sweep_entry(pkg, torch, dev, b16, Ts, 100 if Ts < 4096 else 20,
                                          zipf=zipf if Ts == 4096 else None))
        del b16
        torch.cuda.empty_cache()
        line["sweep"] = sweep
        line["ep_share"] = ep_share_entry(pkg, torch, dev)
    if not args.no_decode_step and not args.no_sweep:
        del layer.copies[1:]
        torch.cuda.empty_cache()
        line["decode_step"] = decode_step_entry(pkg, torch, dev)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch, layer, router, xs[0])
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
