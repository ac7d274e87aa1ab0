"""Throughput of the run-time SDM mixer forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--core-only [--core-input repeated]] [--copy-probe]

Workload: one RunTimeSdm layer forward at B=8, T=2048, d=768, 12 heads of width 64, 1,024 product-key locations
per head, k=8, bf16 activations and weights, float32 memory state, synthetic seeded inputs and Xavier weights.  A
step is one module forward (fused RMSNorm, fused input projection GEMM, SDM core, output map) over the 16,384
tokens, with inputs already resident in HBM; value = 16,384 * K / the wall time of K steps.  Prints one JSON line.

roofline: the SDM core (sdm_rt_forward: plan_kernel and scan_kernel, from the projection outputs to the read-out
before wo) is HBM-bound.  Its algorithmic traffic is 6,168 B per token (kz, qz, V in bf16 =
3 x 1,536 B, gate logits 24 B, read-out 1,536 B) plus 104,544 B of parameters per call: 101,161,056 B at this
shape.  achieved = that / the core's median call time (5 warm calls, then the median of 50, each bracketed by HIP
events on the stream the kernels run on).  traffic = measured HBM bytes per call (rocprofv3 FETCH_SIZE +
WRITE_SIZE summed over the core's kernels, scaled by the same counters' reading for a device copy of known size),
read from profiles/sdm_core_traffic_b8_t2048.txt when present (null otherwise).

config1: the same layer forward at B=1, T=256 in float32 (the reference's CPU-runnable configuration), median of 50
calls.

module: the whole layer is MFMA-bound (79.6 GFLOP per call against 55.2 MB): module.frac = max(bytes / 8 TB/s,
FLOPs / 2.5 PFLOP/s) / module time.  copy_gbs: a 1 GiB device-to-device copy, for context.

cpu_baseline: the float32 torch CPU restatement of the reference forward (oracle/sdm_torch32.py, the reference's
dense chunk algorithm) on the same workload, all host cores, one warm call then best of three; also at B=1, T=256
(B=1, T=256), with the CPU model.  In the same leg the oracle checks the whole models: model.logit_agreement is the
float32 GPU logits of both full-width models (B=1, T=64) against the fp64 oracle (oracle.sdm_fp64.model_forward).

decode: the decode step (sdm_rt_decode_step, one token for each of 64 streams, 12 heads, float32 state carried in
place) timed as a HIP graph of 64 steps replayed 513 times, so the state runs through 32,832 positions; before every
replay the graph's input rows are refilled with the projections of fresh random tokens, so every step addresses new
rows.  us_per_step = replay time / 64 (device time, no host launch cost), reported overall (median) and at positions
0, 1,024, 8,192 and 32,768 to show that the cost of a step does not grow with the position, and again with head 0's
fade set to 0 (us_per_step_head0_fade0).  --no-decode skips it.

model: the whole OneSdmLM forward (logits) at B=8, T=2048, vocabulary 32,768, 12 layers of d=768 with this mixer
(12 heads, M=1,024, k=8): "swiglu" = each layer's per-token step a SwiGLU of hidden 2,048 (the PARTIAL model),
"trained_sdm" = a TrainedSdm of 4,096 slots, one head of width 768, k=16 (the FULL model); bf16 weights and activations,
synthetic seeded weights (the zero-start output maps and tables filled), median of 5 calls after 2 warm; graph_ms
is the same forward replayed from a HIP graph captured at that shape (ForwardGraph), median of 5 replays.
--no-model skips it.

decode_model: the FULL model (the trained_sdm arm above) decoding 64 independent streams, one fresh random token
per stream per step, through 32,832 positions, bf16 weights, float32 state carried in
place; steps run as HIP graphs of 64 (DecodeGraph), the tokens refilled between replays; us_per_step = replay time
/ 64, reported overall (median), as tokens/s (64 / us_per_step) and at positions 0, 1,024, 8,192 and 32,768.
--no-decode-model skips it; --decode-model-steps N shortens it.

train: the backward -- the core's training forward (sdm_rt_forward_train: the forward plus the saved picks, weights,
scores, read and denominators) and backward (sdm_rt_backward) on the layer's bf16 projections, median of 20 calls,
and one RunTimeSdm layer training step (forward + backward under bf16 autocast), median of 10; and the TrainedSdm table
layer of the FULL model (addressing + table read, and sdm_rt_table_backward), median of 20.  --no-train skips it.

--copy-probe runs one 256 MiB device copy before the core calls (the calibration kernel for the traffic counters).
--core-only --core-input repeated times the core on the projections of one repeated token per batch row (the core's
slowest input: every chunk's positions pick the same locations), for profiler runs.
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "RunTimeSdm fwd tokens/sec @B=8,T=2048,d=768 (1 GPU) + % HBM roofline"
B, T, D, H, N_SUB, D_A, K = 8, 2048, 768, 12, 32, 64, 8
HBM_PEAK_GBS = 8000.0
CORE_BYTES_PER_TOKEN = 3 * H * 64 * 2 + H * 2 + H * 64 * 2          # 6,168
CORE_PARAM_BYTES = 2 * H * N_SUB * (D_A // 2) * 4 + H * D_A * 4 + 2 * H * 4 + H * 64 * 4   # keys, addr_b, scale, fade, onorm
BF16_PEAK_FLOPS = 2.5e15
# whole layer: x in and y out (bf16), the four projections and wo (bf16), wg bias and norm weight, core parameters
MODULE_BYTES = B * T * D * 2 * 2 + 4 * D * D * 2 + (D * H * 2 + H * 2) + D * 2 + CORE_PARAM_BYTES
# projections, wo, key scores (2 address sets x 2 halves x 32 sub-keys x 32 dims x 2), sparse write and read
MODULE_FLOPS = B * T * (2 * D * (3 * D + H) + 2 * D * D + 98_304 + 24_960)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def read_traffic():
    path = os.path.join(ROOT, "profiles", "sdm_core_traffic_b8_t2048.txt")
    if not os.path.exists(path):
        return None
    m = re.search(r"^traffic_bytes_per_call:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline():
    """The float32 CPU restatement of the reference forward at the bench shape (and at B=1, T=256), all host
    cores, one warm call then best of three."""
    import torch

    from oracle import sdm_torch32 as R
    from sdmchat_amd import synthetic as S

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    cfg = S.layer_cfg(d=D, heads=H, n_sub=N_SUB, d_a=D_A, k=K)
    p = {n: torch.from_numpy(v) for n, v in S.layer_params(cfg, seed=0).items()}

    def best_of_3(x):
        best = float("inf")
        with torch.no_grad():
            R.forward(x, p, cfg)
            for _ in range(3):
                t0 = time.perf_counter()
                R.forward(x, p, cfg)
                best = min(best, time.perf_counter() - t0)
        return best

    best = best_of_3(torch.from_numpy(S.layer_input(B, T, D, seed=1)))
    best1 = best_of_3(torch.from_numpy(S.layer_input(1, 256, D, seed=1)))
    return {"value": round(B * T / best, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu": _cpu_model(), "b1_t256_tokens_per_s": round(256 / best1, 1),
            "sample": f"full workload B={B} T={T} in float32 (chunk 128), torch {torch.__version__} on the host CPU, "
                      f"1 warm call then best of 3 ({best:.2f} s per call); B=1, T=256 likewise "
                      f"({best1 * 1e3:.1f} ms per call)"}


def logit_agreement(dev, T_agree=64):
    """The whole models' float32 logits on the GPU against the fp64 oracle (oracle.sdm_fp64.model_forward) at full
    width, B=1, T=T_agree: the oracle takes the GPU's picks where two slots' fp64 scores are within 1e-5 (float32
    rounding of the layers' inputs may resolve such near ties the other way)."""
    import numpy as np
    import torch

    from oracle import sdm_fp64 as O
    from sdmchat_amd import synthetic as S

    out = {}
    idx = S.model_tokens(1, T_agree, seed=41)
    for name in ("swiglu", "trained_sdm"):
        m = S.full_model(name)
        p = {n: v.detach().double().numpy() for n, v in m.state_dict().items()}
        m = m.to(dev).eval()
        for mm in m.mems:
            mm.keep_picks = True
        with torch.no_grad():
            got = m(torch.from_numpy(idx).to(dev)).double().cpu().numpy()
        forced = {}
        for i, mm in enumerate(m.mems):
            kk = min(mm.k, min(mm.k, mm.n_sub) ** 2)
            forced[("mem", i)] = tuple(s_[..., :kk].permute(0, 2, 1, 3).reshape(T_agree, mm.h, kk).cpu().numpy()
                                       for s_ in mm.last_picks)
        for i, sd in enumerate(getattr(m, "sdms", [])):
            forced[("sdm", i)] = sd.last_si.cpu().numpy()
        cfg = dict(layers=m.n_layers, heads=m.mems[0].h, d_a=m.mems[0].d_a, k=m.mems[0].k, ffn=m.ffn,
                   adopt_tol=1e-5, adopt_log=[])
        if m.ffn == "sdm":
            cfg.update(sdm_heads=m.sdms[0].h, sdm_d_a=m.sdms[0].d_a, sdm_k=m.sdms[0].k)
        want = O.model_forward(idx, p, cfg, forced=forced)
        scale = np.abs(want).max()
        out[name] = {"max_abs_err_over_scale": float(f"{np.abs(got - want).max() / scale:.3g}"),
                     "top1_agreement": round(float((got.argmax(-1) == want.argmax(-1)).mean()), 4),
                     "ties_taken": int(sum(cfg["adopt_log"]))}
        log(f"logit agreement {name}: {out[name]}")
        del m
        torch.cuda.empty_cache()
    out["workload"] = (f"float32 GPU logits of the full-width models (d 768, 12 layers, vocabulary 32,768) against "
                       f"the fp64 oracle, B=1, T={T_agree}; ties_taken: addresses where the oracle took the GPU's "
                       "pick (fp64 score gap < 1e-5)")
    return out


def decode_bench(m, dev, streams=64, graph_steps=64, replays=513):
    """Device time of sdm_rt_decode_step for `streams` streams of the layer, by position (see the module doc): a HIP
    graph of `graph_steps` steps over static input rows, refilled with fresh random tokens' projections before every
    replay, so every step addresses new rows.  Measured with the layer's fades and again with head 0's fade set to
    0 (its state holds only the last step's writes)."""
    import numpy as np
    import torch

    from sdmchat_amd import core

    gen = torch.Generator(device=dev).manual_seed(7)

    def fresh():
        x = torch.randn(graph_steps * streams, 1, D, generator=gen, device=dev).to(torch.bfloat16)
        return [t[:, 0].reshape(graph_steps, streams, -1) for t in m._project(x, torch.bfloat16)]

    bufs = [t.clone() for t in fresh()]
    out = torch.empty(streams, D, dtype=torch.bfloat16, device=dev)
    ws = core.CoreWorkspace()
    res = {}
    for name, zero_head in (("layer fades", False), ("head 0 fade 0", True)):
        decay = m.decay().detach().clone()
        if zero_head:
            decay[0] = 0.0
        prm = core._params(dev, m.keys1, m.keys2, m.addr_b, m.log_scale, decay, m.onorm_w, None)
        st = m.decode_state(streams, dev)

        def step(t):
            core.decode_step(bufs[0][t], bufs[1][t], bufs[2][t], bufs[3][t], st, keys1=m.keys1, keys2=m.keys2,
                             log_scale=m.log_scale, decay=decay, k=K, out=out, workspace=ws, params=prm)

        for t in range(3):
            step(t)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for t in range(graph_steps):
                step(t)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
        for e0, e1 in evs:
            for b_, f_ in zip(bufs, fresh()):
                b_.copy_(f_)
            e0.record()
            graph.replay()
            e1.record()
        torch.cuda.synchronize()
        us = np.array([e0.elapsed_time(e1) * 1e3 / graph_steps for e0, e1 in evs])
        by_pos = {str(pos): round(float(us[pos // graph_steps]), 2) for pos in (0, 1024, 8192, 32768)
              if pos // graph_steps < replays}
        log(f"decode ({name}): {np.median(us):.2f} us per step (median over {replays} replays), by position {by_pos}")
        res[name] = (round(float(np.median(us)), 2), by_pos)
        del graph
    return {"workload": f"RunTimeSdm decode step: {streams} streams x {H} heads, one fresh random token each per "
                        f"step, float32 state", "us_per_step": res["layer fades"][0],
            "us_per_step_by_position": res["layer fades"][1], "us_per_step_head0_fade0": res["head 0 fade 0"][0],
            "steps_timed": replays * graph_steps,
            "method": f"HIP graph of {graph_steps} steps, replay time / {graph_steps}; inputs refilled with new "
                      "random tokens' projections between replays"}


def model_bench(dev):
    """Whole OneSdmLM forward (logits) for the SwiGLU and the TrainedSdm arms (see the module doc)."""
    import torch

    from sdmchat_amd import ForwardGraph, synthetic as S

    out = {}
    idx = torch.from_numpy(S.model_tokens(B, T, seed=11)).to(dev)
    for name in ("swiglu", "trained_sdm"):
        m = S.full_model(name).to(dev).to(torch.bfloat16).eval()
        with torch.no_grad():
            for _ in range(2):
                m(idx)
            torch.cuda.synchronize()
            ts = []
            for _ in range(5):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                m(idx)
                e1.record()
                torch.cuda.synchronize()
                ts.append(e0.elapsed_time(e1))
        ms = sorted(ts)[2]
        with torch.no_grad():   # the same forward replayed from a HIP graph (ForwardGraph)
            gr = ForwardGraph(m, B, T)
            tg = []
            for _ in range(5):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                gr.run(idx)
                e1.record()
                torch.cuda.synchronize()
                tg.append(e0.elapsed_time(e1))
        gms = sorted(tg)[2]
        out[name] = {"ms": round(ms, 3), "tokens_per_s": round(B * T / (ms * 1e-3), 1), "graph_ms": round(gms, 3),
                     "graph_tokens_per_s": round(B * T / (gms * 1e-3), 1)}
        log(f"model {name}: {ms:.2f} ms per forward, {B * T / (ms * 1e-3) / 1e6:.2f} M tokens/s; "
            f"HIP graph {gms:.2f} ms, {B * T / (gms * 1e-3) / 1e6:.2f} M tokens/s")
        del m, gr
        torch.cuda.empty_cache()
    mf = S.MODEL_FULL
    out["workload"] = (f"OneSdmLM forward (logits): B={B} T={T}, vocabulary {mf['V']}, {mf['layers']} layers, "
                       f"d={mf['d']}, mixer {mf['heads']} heads M={mf['n_sub'] ** 2} k={mf['k']}; swiglu: hidden "
                       f"{mf['mlp_f']}; trained_sdm: 4,096 slots, 1 head, k=16; bf16")
    return out


def decode_model_bench(dev, streams=64, graph_steps=64, total=32768):
    """The FULL model (the trained_sdm arm) decoding `streams` streams, one fresh random token per stream per step,
    through `total` positions (see the module doc)."""
    import numpy as np
    import torch

    from sdmchat_amd import DecodeGraph, synthetic as S

    m = S.full_model("trained_sdm").to(dev).to(torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(13)
    replays = total // graph_steps + 1
    with torch.no_grad():
        st = m.decode_state(streams, dev)
        g = DecodeGraph(m, st, steps=graph_steps)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
        t0 = time.perf_counter()
        for e0, e1 in evs:
            toks = torch.randint(0, m.V, (graph_steps, streams), generator=gen, device=dev)
            e0.record()
            g.run(toks)
            e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    us = np.array([e0.elapsed_time(e1) * 1e3 / graph_steps for e0, e1 in evs])
    by_pos = {str(p): round(float(us[p // graph_steps]), 1) for p in (0, 1024, 8192, 32768) if p <= total}
    steps = replays * graph_steps
    floor = graph_kernel_floor_us(dev)
    log(f"decode (FULL model): {np.median(us):.1f} us per step, {streams * 1e6 / np.median(us):.0f} tokens/s, by "
        f"position {by_pos}; {steps} steps in {wall:.1f} s; a kernel of no work costs {floor:.2f} us in a graph")
    return {"workload": f"FULL OneSdmLM (trained_sdm arm) decode: {streams} streams, one fresh random token per "
                        f"stream per step, {steps} steps, bf16, float32 state ({st.nbytes() / 2 ** 30:.2f} GiB)",
            "us_per_step": round(float(np.median(us)), 1), "tokens_per_s": round(streams * 1e6 / float(np.median(us)), 1),
            "us_per_step_by_position": by_pos, "wall_s": round(wall, 2),
            "method": f"HIP graph of {graph_steps} steps (DecodeGraph), replay time / {graph_steps}",
            "graph_kernel_floor_us": round(floor, 2)}


def graph_kernel_floor_us(dev, n=64, replays=200):
    """The cost of one kernel of (almost) no work inside a HIP graph: n one-element adds captured in one graph,
    replay time / n, best of three runs of `replays` replays (what every launch of a graph-replayed step pays)."""
    import torch

    t = torch.zeros(1, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        t.add_(1.0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(n):
            t.add_(1.0)
    g.replay()
    torch.cuda.synchronize()
    best = 1e9
    for _ in range(3):
        t0 = time.perf_counter()
        for _ in range(replays):
            g.replay()
        torch.cuda.synchronize()
        best = min(best, (time.perf_counter() - t0) / (replays * n))
    return best * 1e6


def train_bench(m, dev, x, kz, qz, V, g, prm, median_call_ms):
    """The backward: the core's training forward (sdm_rt_forward_train) and backward (sdm_rt_backward) on the
    layer's bf16 projections, and one whole layer training step (forward + backward of RunTimeSdm under bf16
    autocast, the reference's training setting)."""
    import torch

    from sdmchat_amd import core

    opts = dict(k=K, read_mode="mean", out_norm=True, read_eps=1e-3, out_norm_eps=1e-2)
    ws_f, ws_b = core.CoreWorkspace(), core.CoreWorkspace()
    state = {}

    def fwd():
        state["r"], state["saved"] = core.core_forward_train(kz, qz, V, g, params=prm, workspace=ws_f, **opts)

    fwd()
    dy = torch.randn(B, T, D, generator=torch.Generator().manual_seed(9)).to(dev)

    def bwd():
        core.core_backward(kz, qz, V, g, state["saved"], dy, params=prm, workspace=ws_b, **opts)

    f_ms = median_call_ms(fwd, n=20, warm=3)
    b_ms = median_call_ms(bwd, n=20, warm=3)
    log(f"train: core forward_train {f_ms * 1e3:.1f} us, core backward {b_ms * 1e3:.1f} us")
    m.train()
    xg = x.detach().clone().requires_grad_(True)
    wgt = torch.randn(B, T, D, generator=torch.Generator().manual_seed(10)).to(dev).to(torch.bfloat16)

    def step():
        with torch.enable_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            y = m(xg)
            (y.float() * wgt.float()).sum().backward()

    s_ms = median_call_ms(step, n=10, warm=2)
    m.eval()
    m.zero_grad(set_to_none=True)
    log(f"train: layer step (forward + backward) {s_ms:.3f} ms")
    # the TrainedSdm table layer of the FULL model: 1 head of width 768, 4,096 slots, k=16, d_a 32
    gen = torch.Generator().manual_seed(12)
    q = torch.randn(B, T, 32, generator=gen).to(dev).to(torch.bfloat16)
    tk1, tk2 = (torch.randn(1, 64, 16, generator=gen).to(dev) for _ in range(2))
    tls = torch.full((1,), 2.0794, device=dev)
    tv = torch.randn(1, 4096, 768, generator=gen).to(dev) * 0.02
    tprm = core._params(dev, tk1, tk2, None, tls, None, None, None)
    tws = core.CoreWorkspace()
    tstate = {}

    def tfwd():
        sl, sc, wt = core.address(q, tk1, tk2, 16, tls, padded=True, params=tprm)
        tstate["p"] = (sl, sc, wt)
        core.table_read(sl, wt, tv, 16, out_dtype=torch.float32)

    tfwd()
    tdy = torch.randn(B, T, 768, generator=gen).to(dev)

    def tbwd():
        sl, sc, wt = tstate["p"]
        core.table_backward(q, sl, wt, sc, tv, tdy, k=16, params=tprm, workspace=tws)

    tf_ms = median_call_ms(tfwd, n=20, warm=3)
    tb_ms = median_call_ms(tbwd, n=20, warm=3)
    log(f"train: table layer forward {tf_ms * 1e3:.1f} us, backward {tb_ms * 1e3:.1f} us")
    return {"core_forward_train_ms": round(f_ms, 4), "core_backward_ms": round(b_ms, 4),
            "layer_step_ms": round(s_ms, 4), "layer_step_tokens_per_s": round(B * T / (s_ms * 1e-3), 1),
            "table_forward_ms": round(tf_ms, 4), "table_backward_ms": round(tb_ms, 4),
            "workload": f"RunTimeSdm layer training step at B={B} T={T} d={D}, 12 heads, M=1,024, k=8, bf16 autocast; "
                        "core = sdm_rt_forward_train / sdm_rt_backward on the bf16 projections; table = the "
                        "TrainedSdm layer between wq and wo (1 head of 768, 4,096 slots, k=16): sdm_rt_address + "
                        "sdm_rt_table_read, and sdm_rt_table_backward"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--core-only", action="store_true", help="time only the SDM core (for profiler runs)")
    ap.add_argument("--core-input", choices=("varied", "repeated"), default="varied",
                    help="with --core-only: the layer input, or one repeated token per batch row")
    ap.add_argument("--copy-probe", action="store_true", help="run one 256 MiB device copy first (counter calibration)")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode-step measurement")
    ap.add_argument("--decode-replays", type=int, default=513, help="graph replays of the decode-step measurement")
    ap.add_argument("--no-model", action="store_true", help="skip the whole-model measurement")
    ap.add_argument("--no-decode-model", action="store_true", help="skip the whole-model decode measurement")
    ap.add_argument("--decode-model-only", action="store_true", help="only the whole-model decode (profiler runs)")
    ap.add_argument("--decode-model-steps", type=int, default=32768, help="positions the whole-model decode runs")
    ap.add_argument("--model-only", action="store_true", help="only the whole-model measurement (for profiler runs)")
    ap.add_argument("--no-train", action="store_true", help="skip the backward measurement")
    ap.add_argument("--train-only", action="store_true", help="only the backward measurement (for profiler runs)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU only (asked for {a.gpus}); the mixer runs on one GPU here, so no figure at "
              "several GPUs is produced",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from sdmchat_amd import RunTimeSdm, core, synthetic as S

    dev = torch.device("cuda:0")
    if a.model_only:
        print(json.dumps({"model": model_bench(dev)}), flush=True)
        return
    if a.decode_model_only:
        print(json.dumps({"decode_model": decode_model_bench(dev, total=a.decode_model_steps)}), flush=True)
        return
    cfg = S.layer_cfg(d=D, heads=H, n_sub=N_SUB, d_a=D_A, k=K)
    params = S.layer_params(cfg, seed=0)
    m = RunTimeSdm(D, heads=H, n_sub=N_SUB, d_a=D_A, k=K, decays=tuple(float(v) for v in params["decays_fixed"]))
    m.load_state_dict({n: torch.from_numpy(v) for n, v in params.items()}, strict=True)
    m = m.to(dev).eval()
    x = torch.from_numpy(S.layer_input(B, T, D, seed=1)).to(dev).to(torch.bfloat16)
    if a.core_input == "repeated":
        if not a.core_only:
            sys.exit("--core-input repeated times the core only (--core-only)")
        x = x[:, :1].expand(B, T, D).contiguous()

    with torch.no_grad():
        kz, qz, V, g = m._project(x, torch.bfloat16)
        prm = core._params(dev, m.keys1, m.keys2, m.addr_b, m.log_scale, m.decay(), m.onorm_w, None)
        ws = core.CoreWorkspace()
        r_out = torch.empty(B, T, D, dtype=torch.bfloat16, device=dev)

        def core_call():
            core.core_forward(kz, qz, V, g, keys1=m.keys1, keys2=m.keys2, log_scale=m.log_scale, decay=m.decay(),
                              k=K, out=r_out, workspace=ws, params=prm)

        if a.copy_probe:
            src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
            dst = torch.empty_like(src)
            dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst

        def median_call_ms(fn, n=50, warm=5):
            for _ in range(warm):
                fn()
            torch.cuda.synchronize()
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
            for e0, e1 in evs:
                e0.record()
                fn()
                e1.record()
            torch.cuda.synchronize()
            ts = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
            return ts[n // 2]

        def timed(fn, steps, warmup):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            torch.cuda.synchronize()
            return time.perf_counter() - t0

        if a.train_only:
            print(json.dumps({"train": train_bench(m, dev, x, kz, qz, V, g, prm, median_call_ms)}), flush=True)
            return
        core_ms = median_call_ms(core_call)
        log(f"core: {core_ms * 1e3:.1f} us per call (median of 50)")
        if a.core_only:
            print(json.dumps({"core_ms": core_ms}))
            return
        mod_ms = median_call_ms(lambda: m(x))
        wall = timed(lambda: m(x), a.steps, a.warmup)
        x1 = torch.from_numpy(S.layer_input(1, 256, D, seed=2)).to(dev)   # config 1: B=1, T=256, float32
        c1_ms = median_call_ms(lambda: m(x1))
        big = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        big2 = torch.empty_like(big)
        copy_ms = median_call_ms(lambda: big2.copy_(big), n=10, warm=2)
        del big, big2
        decode = None if a.no_decode else decode_bench(m, dev, replays=a.decode_replays)
        train = None if a.no_train else train_bench(m, dev, x, kz, qz, V, g, prm, median_call_ms)
        model = None if a.no_model else model_bench(dev)
        decode_model = None if a.no_decode_model else decode_model_bench(dev, total=a.decode_model_steps)

    ms_per_step = wall * 1e3 / a.steps
    tokens = B * T
    core_bytes = CORE_BYTES_PER_TOKEN * tokens + CORE_PARAM_BYTES
    achieved = core_bytes / (core_ms * 1e-3) / 1e9
    rec = {
        "metric": METRIC,
        "value": round(tokens / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs, Xavier-uniform weights, N(0,1) sub-keys, fades U(0.9, 0.999))",
        "config": {"workload": "RunTimeSdm layer forward", "batch": B, "seq_len": T, "d": D, "heads": H,
                   "head_dim": D // H, "locations_per_head": N_SUB * N_SUB, "top_k": K,
                   "activations": "bf16", "memory_state": "fp32"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "kernel": "SDM core (sdm_rt_forward)", "algorithmic_bytes": core_bytes,
                     "ms_per_call": round(core_ms, 5)},
        "core": {"ms": round(core_ms, 5), "tokens_per_s": round(tokens / (core_ms * 1e-3), 1)},
        "module": {"ms": round(mod_ms, 5), "bound": "mfma", "bytes": MODULE_BYTES, "flops": MODULE_FLOPS,
                   "frac": round(max(MODULE_BYTES / (HBM_PEAK_GBS * 1e9), MODULE_FLOPS / BF16_PEAK_FLOPS)
                                 / (mod_ms * 1e-3), 4)},
        "copy_gbs": round(2 * (1 << 30) / (copy_ms * 1e-3) / 1e9, 1),
        "config1": {"workload": "RunTimeSdm layer forward, B=1 T=256, float32 activations and weights",
                    "ms": round(c1_ms, 5), "tokens_per_s": round(256 / (c1_ms * 1e-3), 1)},
    }
    if decode is not None:
        rec["decode"] = decode
    if model is not None:
        rec["model"] = model
    if decode_model is not None:
        rec["decode_model"] = decode_model
    if train is not None:
        rec["train"] = train
    if not a.no_cpu:
        log("cpu baseline ...")
        rec["cpu_baseline"] = cpu_baseline()
        if model is not None:   # the oracle as the checker of the whole model's logits
            rec["model"]["logit_agreement"] = logit_agreement(dev)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
