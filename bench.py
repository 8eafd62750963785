"""Benchmark of the thinker MoE block on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Headline workload: one MoE block prefill of 512 tokens (hidden 2048, 64 routed experts of 1408 plus a
shared expert, softmax top-6, router bias ~ N(0, 0.5) for ragged expert loads). A step is the whole
block on inputs already resident in HBM: RMSNorm -> router -> align -> grouped gate/up -> down ->
combine + residual, replayed from one hipGraph. `value` is tokens/s over exactly K timed steps.

Also measured and reported under "extra": the 2048-token Zipf prefill; the headline block with int8 experts
(fp32 row scales); the block on the row layouts (no prefill copies); the full 28-layer synthetic decode
step (+ LM head) in one hipGraph; decode of 1 token (bf16) and int8 decode at batch 1/2/4/8 through 28
distinct layers (cold: every layer's experts read from HBM), per layer and per kernel; the Talker path (a
24-layer Qwen2-0.5B-shaped LLM decode step and its rotary / decode attention and silu_mul kernels); and the
ingestion of one MoE layer's experts from safetensors shards into the stacked bf16 / int8 layout. The
roofline of the dominant kernel (prefill gate/up) is its algorithmic bytes over its average duration from HIP
events on its own stream; the CPU baseline is the reference's torch path (the per-expert bf16 loop) on all
512 tokens of the headline workload on this host.
"""
import argparse
import csv
import glob
import json
import os
import platform
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "ming-voice_amd"), ROOT]

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline line only (no extra workloads)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="",
                    help="comma list of extra workloads to run (decode,int8,zipf,full,hybrid,hybrid_prefill,talker,ingest)")
    ap.add_argument("--no-pmc", action="store_true", help="skip the rocprofv3 counter passes (traffic = null)")
    ap.add_argument("--pmc-probe", action="store_true", help=argparse.SUPPRESS)
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def graph_of(fn, stream):
    """Captures fn() once into a hipGraph on `stream` (after one eager warm call). `stream` first waits for the
    current stream: the warm call reads (and writes) tensors the current stream made, and the caching allocator may
    have handed them memory whose previous owner that stream's queued kernels still read."""
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    return g


def time_graph(g, stream, reps, warmup=2):
    """Average ms per replay, from HIP events recorded on the replay stream (ordered after the current stream's
    work, and the current stream after the replays)."""
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        stream.synchronize()
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        e1.synchronize()
    torch.cuda.current_stream().wait_stream(stream)
    return e0.elapsed_time(e1) / reps


def kernel_ms(fn, stream, reps=20):
    """Average duration of the launch(es) in fn: `reps` copies captured in one graph, timed with events."""
    g = graph_of(lambda: [fn() for _ in range(reps)], stream)
    return time_graph(g, stream, 5) / reps


# ----------------------------------------------------------------------------------------------- prefill

class copies:
    """Sets fused_moe.PREFILL_COPIES for a block of calls: "registered" (the prefill GEMMs read the copies that
    fused_moe.prefill_copies registered for the stacks, found by the calls themselves) or "off" (the stacks)."""

    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        import fused_moe
        self.prev, fused_moe.PREFILL_COPIES = fused_moe.PREFILL_COPIES, self.mode

    def __exit__(self, *exc):
        import fused_moe
        fused_moe.PREFILL_COPIES = self.prev
        return False


def prefill_setup(b, n, bias, seed, slabs=True, int8=False):
    """The prefill block on n tokens; slabs: the GEMMs read the prefill copies of the stacks registered with
    fused_moe.prefill_copies (a load-time layout step), found by the calls themselves; else the stacks. int8: the
    experts are b["q_gu"] / b["q_d"] with row scales b["s_gu"] / b["s_d"]."""
    import fused_moe
    import workloads as W
    wg, wd = (b["q_gu"], b["q_d"]) if int8 else (b["w_gu"], b["w_d"])
    sg, sd = (b["s_gu"], b["s_d"]) if int8 else (None, None)
    x = W.tokens(n, seed=seed, device="cuda")
    E1, I, H = b["w_gu"].shape[0], b["w_d"].shape[-1], b["w_d"].shape[1]
    sc = fused_moe.PrefillScratch(n, W.TOP_K + 1, E1, H, I, x.device, block=True, w_dtype=wg.dtype)
    st = {"xn": sc.xn, "ids": sc.ids, "wts": sc.wts}

    mode = "registered" if slabs else "off"

    def step():  # the whole block: RMSNorm + router + select + align + gate/up + down + combine (+ x)
        with copies(mode):
            return fused_moe.moe_block_prefill(x, b["norm_w"], W.EPS, b["w32"], wg, wd, top_k=W.TOP_K, bias=bias,
                                               scoring="softmax", s_gu=sg, s_d=sd, scratch=sc)[0]

    step()
    torch.cuda.synchronize()
    with copies(mode):
        st["w_gu_slabs"], st["w_d_slabs"] = fused_moe._copies_for(wg, wd)
    st["mode"] = mode
    st["experts"] = (wg, wd, sg, sd)
    return x, sc, st, step


def prefill_metrics(b, n, bias, steps, warmup, stream, seed=70, slabs=True, int8=False):
    import fused_moe
    import _mingmoe
    import workloads as W
    x, sc, st, step = prefill_setup(b, n, bias, seed, slabs, int8)
    wg, wd, sg, sd = st["experts"]
    g = graph_of(step, stream)
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            g.replay()
        stream.synchronize()
        t0 = time.perf_counter()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            g.replay()
        e1.record(stream)
        busy = read_clocks()  # the replays are still running: the clocks of the timed region
        e1.synchronize()
        wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    ids = st["ids"]
    counts = torch.bincount(ids.reshape(-1), minlength=b["w_gu"].shape[0]).cpu()
    used = int((counts > 0).sum())
    P = ids.numel()

    def phase(p):
        def run():
            with copies(st["mode"]):
                fused_moe.fused_moe_prefill(st["xn"], wg, wd, ids, st["wts"], s_gu=sg, s_d=sd, residual=x, scratch=sc,
                                            phases=p, align=False)
        return run
    gu_ms = kernel_ms(phase(_mingmoe.MM_PHASE_GATE_UP), stream)
    dn_ms = kernel_ms(phase(_mingmoe.MM_PHASE_DOWN), stream)
    cb_ms = kernel_ms(phase(_mingmoe.MM_PHASE_COMBINE), stream)
    H, I = W.HIDDEN, W.INTER
    es, sb = (1, sg.element_size()) if int8 else (2, 0)  # weight bytes per element, scale bytes per row
    gu_bytes = used * 2 * I * (H * es + sb) + n * H * 2 + P * I * 2
    dn_bytes = used * H * (I * es + sb) + P * I * 2 + P * H * 2
    flops = P * W.flops_per_pair()
    moe_ms = gu_ms + dn_ms
    return {
        "tokens": n, "ms_per_step": ms, "tokens_per_s": n / ms * 1e3, "wall_s": wall,
        "experts_used": used, "top3_share": float(counts[:-1].sort(descending=True).values[:3].sum() / P),
        "gate_up_us": gu_ms * 1e3, "down_us": dn_ms * 1e3, "combine_us": cb_ms * 1e3,
        "gate_up_GBs": gu_bytes / gu_ms / 1e6, "down_GBs": dn_bytes / dn_ms / 1e6, "gate_up_bytes": gu_bytes,
        "mfma_pct": flops / (moe_ms * 1e-3) / (MFMA_BF16_PEAK_TFLOPS * 1e12) * 100,
        "hbm_pct_weights": used * W.expert_bytes(int8=int8, scale_bytes=sb) / (moe_ms * 1e-3) / (HBM_PEAK_GBS * 1e9)
        * 100,
        "weights": f"int8 + {'fp32' if sb == 4 else 'bf16'} row scales" if int8 else "bf16",
        "mode": st["mode"],
        "gate_up_weights": "slab copy" if st["w_gu_slabs"] is not None else "rows",
        "down_weights": "slab copy" if st["w_d_slabs"] is not None else "rows",
        "clocks_under_load": busy,
    }


def engine_call_metrics(b, n, bias, stream, seed=70, reps=20):
    """The reference engine's own prefill call, unchanged (engine.py:300-310): fused_moe_prefill(x, w_gu, w_d, ids,
    wts) on the block's stacks, with no layout argument and no scratch, on the normalised rows and routing of the
    headline workload. The call finds the prefill copies registered for the stacks; `reps` calls in one graph."""
    import fused_moe
    import fused_ops
    import workloads as W
    x = W.tokens(n, seed=seed, device="cuda")
    xn = fused_ops.rms_norm(x, b["norm_w"], W.EPS)
    ids, wts, _ = fused_ops.route(xn, b["w32"], bias, top_k=W.TOP_K, scoring="softmax")
    out = {}
    for mode in ("registered", "off"):
        with copies(mode):
            ms = kernel_ms(lambda: fused_moe.fused_moe_prefill(xn, b["w_gu"], b["w_d"], ids, wts), stream, reps)
            found = fused_moe._copies_for(b["w_gu"], b["w_d"])
        out[mode] = {"us": ms * 1e3, "tokens_per_s": n / ms * 1e3, "copies_found": [c is not None for c in found]}
    return {"tokens": n, "call": "fused_moe_prefill(x, w_gu, w_d, ids, wts)", "with_copies": out["registered"],
            "rows": out["off"]}


# ------------------------------------------------------------------------------- HBM traffic (counters)

PROBE_LAUNCHES = 5
COPY_BYTES = 512 << 20  # calibration copy: reads and writes this many bytes, twice the last-level cache


def pmc_probe():
    """Child run under `rocprofv3 --pmc <counter>`: the headline gate/up kernel PROBE_LAUNCHES times on the
    512-token workload, then a plain device copy of COPY_BYTES as many times (counter calibration)."""
    import fused_moe
    import _mingmoe
    import workloads as W
    _mingmoe.load()
    b = W.block(seed=0, device="cuda")
    fused_moe.prefill_copies(b["w_gu"], b["w_d"])
    x, sc, st, step = prefill_setup(b, 512, W.ragged_bias(device="cuda"), 70)
    with copies("registered"):
        for _ in range(PROBE_LAUNCHES):
            fused_moe.fused_moe_prefill(st["xn"], b["w_gu"], b["w_d"], st["ids"], st["wts"], residual=x, scratch=sc,
                                        phases=_mingmoe.MM_PHASE_GATE_UP, align=False)
    torch.cuda.synchronize()
    del b
    src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(PROBE_LAUNCHES):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("[probe] done", flush=True)


def _counter_per_dispatch(path, counter):
    """{kernel name: [counter value of each dispatch]} from a rocprofv3 counter_collection.csv."""
    out = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") == counter:
                out.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return out


def pmc_traffic(timeout=90):
    """HBM bytes per launch of the gate/up kernel: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) from two
    rocprofv3 --pmc passes over pmc_probe(), each scaled by bytes / counter of the calibration copy."""
    tool = shutil.which("rocprofv3")
    if tool is None:
        return None, {"error": "rocprofv3 not found"}
    detail = {}
    total = 0.0
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out = tempfile.mkdtemp(prefix="mm_pmc_")
        cmd = ["timeout", "-s", "KILL", str(timeout), tool, "--pmc", counter, "--output-format", "csv", "-d", out,
               "-o", "pmc", "--", sys.executable, os.path.abspath(__file__), "--pmc-probe"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            shutil.rmtree(out, ignore_errors=True)
            return None, {"error": f"{counter} pass exited {r.returncode} without counters", "stderr": r.stderr[-400:]}
        per = _counter_per_dispatch(files[0], counter)
        shutil.rmtree(out, ignore_errors=True)
        gu = [v for k, vs in per.items() if "prefill_gate_up_kernel" in k for v in vs]
        cp = [v for k, vs in per.items() if "copy" in k.lower() for v in vs]
        if not gu or not cp:
            return None, {"error": f"{counter}: kernels not found in {sorted(per)}"}
        gu_kib, cp_kib = sum(gu) / len(gu), sum(cp) / len(cp)
        factor = COPY_BYTES / (cp_kib * 1024.0)
        detail[counter] = {"gate_up_KiB": gu_kib, "copy_KiB": cp_kib, "copy_bytes": COPY_BYTES, "factor": factor,
                           "bytes": gu_kib * 1024.0 * factor}
        total += gu_kib * 1024.0 * factor
    return total, detail


# ------------------------------------------------------------------------------------------------ decode

def median_graph_ms(g, stream, reps=20, runs=5):
    return sorted(time_graph(g, stream, reps) for _ in range(runs))[runs // 2]


def decode_metrics(blocks, n, stream, int8=False, seed=40):
    """Decode of n tokens through len(blocks) distinct MoE blocks chained (layer l's output is layer l+1's
    input), every block's experts in memory of their own: the 28 layers' active experts (28 x 121 MB in bf16,
    28 x 61 MB in int8 for one token) far exceed the 256 MB last-level cache, so every expert byte of a layer
    comes from HBM, as in a real forward pass. Per layer (graph replays, median of 5 timings): the fused
    block (moe_block_decode: router + norm, selection, gate/up, down + combine), the unfused chain
    (rms_norm -> moe_route -> fused_moe_decode), and each MoE kernel alone (its launches over the 28 layers
    in one graph, on the inputs the chain gave each layer). Bytes: each layer's realised distinct experts."""
    import fused_moe
    import fused_ops
    import _mingmoe
    import workloads as W
    L, dev = len(blocks), "cuda"
    H, I, E, NK = W.HIDDEN, W.INTER, W.EXPERTS, W.TOP_K + 1
    x0 = W.tokens(n, seed=seed + n, device=dev)

    def experts(b):
        return (b["q_gu"], b["q_d"], b["s_gu"], b["s_d"]) if int8 else (b["w_gu"], b["w_d"], None, None)

    logits = torch.empty(n, E, device=dev)
    ids = torch.empty(n, NK, device=dev, dtype=torch.long)
    wts = torch.empty(n, NK, device=dev)
    a_buf = torch.empty(n * NK, I, device=dev, dtype=torch.bfloat16)

    def fused():
        h = x0
        for b in blocks:
            wg, wd, sg, sd = experts(b)
            h = fused_moe.moe_block_decode(h, b["norm_w"], W.EPS, b["w32"], wg, wd, top_k=W.TOP_K, s_gu=sg, s_d=sd,
                                           logits=logits, ids=ids, wts=wts, a_buf=a_buf)[0]
        return h

    def unfused():
        h = x0
        for b in blocks:
            wg, wd, sg, sd = experts(b)
            xn = fused_ops.rms_norm(h, b["norm_w"], W.EPS)
            fused_ops.moe_route(xn, b["w32"], None, 1, 1, W.TOP_K, 1.0, logits, ids, wts, scoring="softmax")
            h = fused_moe.fused_moe_decode(xn, wg, wd, ids, wts, a_buf=a_buf, s_gu=sg, s_d=sd, residual=h)
        return h

    ms = median_graph_ms(graph_of(fused, stream), stream) / L
    ms_unfused = median_graph_ms(graph_of(unfused, stream), stream) / L
    # each layer's kernel inputs, from one eager pass of the unfused chain
    per = []
    h = x0
    for b in blocks:
        xn = fused_ops.rms_norm(h, b["norm_w"], W.EPS)
        li, lw = torch.empty_like(ids), torch.empty_like(wts)
        fused_ops.moe_route(xn, b["w32"], None, 1, 1, W.TOP_K, 1.0, logits, li, lw, scoring="softmax")
        per.append({"xn": xn, "ids": li, "wts": lw, "res": h, "a": torch.empty_like(a_buf),
                    "out": torch.empty(n, H, device=dev, dtype=torch.bfloat16)})
        wg, wd, sg, sd = experts(b)
        h = fused_moe.fused_moe_decode(xn, wg, wd, li, lw, s_gu=sg, s_d=sd, residual=h)

    def phase(p):
        def run():
            for b, q in zip(blocks, per):
                wg, wd, sg, sd = experts(b)
                fused_moe.fused_moe_decode(q["xn"], wg, wd, q["ids"], q["wts"], a_buf=q["a"], out=q["out"], s_gu=sg,
                                           s_d=sd, residual=q["res"], phases=p)
        return run
    gu_ms = median_graph_ms(graph_of(phase(_mingmoe.MM_PHASE_GATE_UP), stream), stream) / L
    dn_ms = median_graph_ms(graph_of(phase(_mingmoe.MM_PHASE_DOWN), stream), stream) / L
    uniq = sum(int(torch.unique(q["ids"]).numel()) for q in per) / L  # distinct experts per layer
    es, sb = (1, 2) if int8 else (2, 0)
    gu_bytes = uniq * (2 * I * H * es + 2 * I * sb)
    dn_bytes = uniq * (H * I * es + H * sb)
    moe_bytes = gu_bytes + dn_bytes
    return {
        "tokens": n, "int8": int8, "layers": L, "cold": True, "unique_experts_per_layer": uniq,
        "us_per_layer": ms * 1e3, "us_per_token_per_layer": ms * 1e3 / n, "us_per_layer_unfused": ms_unfused * 1e3,
        "gate_up_us": gu_ms * 1e3, "down_us": dn_ms * 1e3, "moe_bytes_per_layer": moe_bytes,
        "gate_up_TBs": gu_bytes / gu_ms / 1e9, "down_TBs": dn_bytes / dn_ms / 1e9,
        "moe_TBs": moe_bytes / (gu_ms + dn_ms) / 1e9, "layer_TBs": moe_bytes / ms / 1e9,
        "moe_hbm_pct": moe_bytes / ((gu_ms + dn_ms) * 1e-3) / (HBM_PEAK_GBS * 1e9) * 100,
        "layer_hbm_pct": moe_bytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9) * 100,
    }


# ------------------------------------------------------------------------------------- full decode step

def full_decode_metrics(step, stream):
    """The synthetic thinker decode step (workloads.ThinkerDecodeStep: 28 x (RMSNorm fused into the q|k|v GEMV
    -> o projection + residual -> MoE block) -> final RMSNorm + LM head 2048 -> 126464, batch 1) in one
    hipGraph, and its 28 MoE blocks alone (median of 5 timings), every layer's experts distinct memory."""
    import workloads as W
    layers = len(step.L)
    ms = median_graph_ms(graph_of(step, stream), stream)
    moe_ms = median_graph_ms(graph_of(step.moe_only, stream), stream)
    total = step.bytes_per_step()
    moe_layer_bytes = (W.TOP_K + 1) * W.expert_bytes() + W.EXPERTS * W.HIDDEN * 4
    return {"layers": layers, "us_per_token": ms * 1e3, "bytes_per_token": total, "TBs": total / ms / 1e9,
            "hbm_pct": total / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9) * 100,
            "moe_us_per_layer": moe_ms * 1e3 / layers, "moe_layer_bytes": moe_layer_bytes,
            "moe_TBs": moe_layer_bytes * layers / moe_ms / 1e9}


def hybrid_decode_metrics(stream, layers=28, pos=456):
    """One decode token of the synthetic hybrid thinker (workloads.HybridThinkerStep: 21 KDA + 7 MLA layers, each
    with its MoE block, final norm + LM head) replayed from one hipGraph, and the same with the KDA cores as the
    five-call chain (`us_per_token_kda_chain`), and on int8 experts (fp32 row scales, `int8`). Every replay
    advances the position on
    the device: one eager call at pos, then replays at pos + 1, pos + 2, ...; the timed ones (5 x 20 after 2
    warm-up replays each) lie in pos + 3 .. pos + 110 of a 1024-row cache, mean pos + 56.5 (512.5 by default)."""
    import workloads as W
    step = W.HybridThinkerStep(layers, "cuda", pos=pos)
    torch.cuda.synchronize()
    ms = median_graph_ms(graph_of(step, stream), stream)
    total = step.bytes_per_step(pos + 56)
    kda = sum(p["kind"] == "kda" for p in step.L)
    # the same step with each KDA core as the five-call chain (short_conv, the f / g projections,
    # fused_recurrent_kda, rms_norm_gated) instead of kda_decode_step's one kernel, same process and box
    step.fused_kda = False
    ms_chain = median_graph_ms(graph_of(step, stream), stream)
    out = {"layers": layers, "kda_layers": kda, "mla_layers": layers - kda, "positions": [pos + 3, pos + 110],
           "us_per_token": ms * 1e3, "bytes_per_token": total, "TBs": total / ms / 1e9,
           "hbm_pct": total / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9) * 100, "us_per_token_kda_chain": ms_chain * 1e3}
    # the same step on int8 experts with fp32 row scales (the reference's int8 stacks), same masters
    step.fused_kda = True
    step.use_int8_experts(torch.float32)
    step.pos.fill_(pos)
    ms8 = median_graph_ms(graph_of(step, stream), stream)
    total8 = step.bytes_per_step(pos + 56)
    out["int8"] = {"us_per_token": ms8 * 1e3, "bytes_per_token": total8, "TBs": total8 / ms8 / 1e9,
                   "hbm_pct": total8 / (ms8 * 1e-3) / (HBM_PEAK_GBS * 1e9) * 100}
    del step
    torch.cuda.empty_cache()
    return out


def hybrid_prefill_metrics(stream, layers=28, pos=512, lengths=(32, 128, 512)):
    """A prompt of T tokens through the synthetic hybrid thinker (thinker_step.FastThinkerStep.prefill, the engine's
    _prefill: per layer the mixer over the T rows — the projection GEMMs, the short convolutions and the KDA
    recurrence, or the causal MLA attention over the cache — then the prefill MoE block; the head on the last
    token), captured in one hipGraph per T and replayed at position 512 of a 2048-row cache (the position set back
    before each replay; the layer states keep evolving, which changes no amount of work): median of 5 timed
    replays after one, in ms and prompt tokens/s; then the same on int8 experts (fp32 row scales). The expert
    stacks take the registered prefill copies."""
    import workloads as W
    step = W.HybridThinkerStep(layers, "cuda", pos=pos, max_len=2048, seed=5000)
    out = {"layers": layers, "kda_layers": sum(p["kind"] == "kda" for p in step.L), "pos": pos}
    _prompts(step, stream, pos, lengths, out)
    # the same prompts on int8 experts with fp32 row scales (the reference's int8 stacks), same masters
    step.use_int8_experts(torch.float32)
    out["int8"] = {}
    _prompts(step, stream, pos, lengths, out["int8"])
    del step
    torch.cuda.empty_cache()
    return out


def _prompts(step, stream, pos, lengths, out):
    for T in lengths:
        ids = (torch.arange(T, device="cuda") * 7919 + 11) % step.embed.shape[0]
        step.pos.fill_(pos)
        g = graph_of(lambda: step.fast.prefill(ids), stream)
        ts = []
        for _ in range(6):
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                step.pos.fill_(pos)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                g.replay()
                e1.record(stream)
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        torch.cuda.current_stream().wait_stream(stream)
        ms = sorted(ts[1:])[2]
        out[f"T{T}"] = {"ms": ms, "tokens_per_s": T / ms * 1e3}
        del g


# ------------------------------------------------------------------------------------------- Talker path

def talker_metrics(stream, layers=24, max_len=1024, pos=512):
    """The Talker's per-token work on the HIP kernels: one decode step of a Qwen2-0.5B-shaped Talker LLM
    (FastQwen2Step: 24 layers, hidden 896, 14 query / 2 KV heads of 64, intermediate 4864) at position 512
    of a 1024-position cache, replayed from one hipGraph; the per-latent tail (FastTail: 10 CFG steps of a
    4-block DiT of hidden 1024, a 2-block aggregator, the stop head) from one hipGraph; and per kernel (20
    launches in one graph): the decode
    attention at that position, the rotary attention of a DiT block (2 x 3 tokens) and of an aggregator
    block (1 x 2 tokens), 16 heads of 64, and silu_mul over 4864."""
    import fast_talker as FT
    import workloads as W
    dev = "cuda"
    llm = W.TalkerLLM(layers=layers, max_len=max_len, seed=3000, device=dev)
    llm.fill_cache(pos, seed=3001)
    fs = FT.FastQwen2Step(llm)
    x = W.normal((1, 1, W.TALKER_HIDDEN), 0.1, 3002, dev)
    p = torch.tensor([pos], device=dev)
    g = graph_of(lambda: fs(x, p), stream)  # every replay rewrites cache row pos with the same values
    step_ms = time_graph(g, stream, 20)
    nh, nkv, hd = llm.nh, llm.nkv, llm.hd
    qkv = W.normal((1, (nh + 2 * nkv) * hd), 1.0, 3003, dev)
    out = torch.empty(1, nh * hd, device=dev, dtype=torch.bfloat16)
    ws = FT.decode_attn_workspace(nh, hd, max_len, dev)
    kc, vc = llm.k[0], llm.v[0]
    attn_ms = kernel_ms(lambda: FT.qwen_decode_attn(qkv, kc, vc, p, llm.inv_freq, out, max_len, hd ** -0.5, nh,
                                                    nkv, hd, workspace=ws), stream)
    rope = {}
    for name, (B, S) in (("dit", (2, 3)), ("aggregator", (1, 2))):
        q = W.normal((B, S, 3 * 1024), 1.0, 3004 + S, dev)
        ang = torch.rand(S, 32, device=dev) * 6.283
        c, s_ = ang.cos().contiguous(), ang.sin().contiguous()
        rope[name] = kernel_ms(lambda: FT.rope_attn(q, c, s_, 16), stream) * 1e3
    gu = W.normal((1, 2 * W.TALKER_INTER), 1.0, 3006, dev)
    act = torch.empty(1, W.TALKER_INTER, device=dev, dtype=torch.bfloat16)
    silu_ms = kernel_ms(lambda: FT.silu_mul(gu, act), stream)
    H, I = W.TALKER_HIDDEN, W.TALKER_INTER
    w_bytes = layers * ((nh + 2 * nkv) * hd * H + H * nh * hd + 2 * I * H + H * I) * 2
    kv_bytes = 2 * nkv * (pos + 1) * hd * 2
    del g, fs, llm
    # the per-latent tail: 10 CFG flow-matching steps of a 4-block DiT (hidden 1024) + 2-block aggregator
    tk = W.TalkerTail(seed=3100, device=dev)
    ft = FT.FastTail(tk, tk.ts, tk.dts, tk.cfg_strength)
    ins = [W.normal(shape, 1.0, 3110 + i, dev) for i, shape in enumerate(((1, 1, H), (1, 1, 64), (1, 1, 64)))]
    gt = graph_of(lambda: ft(*ins), stream)
    tail_ms = time_graph(gt, stream, 20)
    del gt, ft, tk
    return {"layers": layers, "pos": pos, "max_len": max_len, "step_us": step_ms * 1e3, "tail_us": tail_ms * 1e3,
            "step_bytes": w_bytes + layers * kv_bytes, "step_TBs": (w_bytes + layers * kv_bytes) / step_ms / 1e9,
            "decode_attn_us": attn_ms * 1e3, "decode_attn_kv_bytes": kv_bytes,
            "rope_attn_dit_us": rope["dit"], "rope_attn_aggregator_us": rope["aggregator"],
            "silu_mul_us": silu_ms * 1e3}


# ------------------------------------------------------------------------------------- expert ingestion

def ingest_metrics(n_experts=64, hidden=2048, inter=1408, threads=4, ref_threads=8):
    """One thinker MoE layer's experts (64 routed + shared, bf16, 1.125 GB over 4 safetensors shards in a
    temporary directory, so the reads come from the page cache) ingested into a bf16 stack and an int8 stack
    (bf16 scales) with expert_load.load_stacked_experts; next to them the reference's method on the same
    files (direct_load.py:109-131 + engine.py:130-135: threads pread each tensor into a bytearray, copy it
    to the GPU from pageable memory, and quantise it there), and a pinned host-to-device copy of 1 GiB (the
    link's practical ceiling)."""
    import fused_moe
    import expert_load as EL
    from workloads import expert_tensors, write_checkpoint
    from concurrent.futures import ThreadPoolExecutor
    dev = torch.device("cuda")
    pfx = "model.layers.1.mlp"
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR")) as tmp:
        t = expert_tensors(pfx, n_experts, hidden, inter, seed=4000)
        root = write_checkpoint(os.path.join(tmp, "ck"), t, shards=4, extra=False)
        nbytes = sum(v.numel() * v.element_size() for v in t.values())
        del t
        E1 = n_experts + 1
        bf = {"w_gu": torch.empty(E1, 2 * inter, hidden, dtype=torch.bfloat16, device=dev),
              "w_d": torch.empty(E1, hidden, inter, dtype=torch.bfloat16, device=dev)}
        q8 = {"q_gu": torch.empty(E1, 2 * inter, hidden, dtype=torch.int8, device=dev),
              "q_d": torch.empty(E1, hidden, inter, dtype=torch.int8, device=dev),
              "s_gu": torch.empty(E1, 2 * inter, dtype=torch.bfloat16, device=dev),
              "s_d": torch.empty(E1, hidden, dtype=torch.bfloat16, device=dev)}
        idx = EL.checkpoint_index(root)

        def timed(fn, reps=3):
            fn()
            torch.cuda.synchronize()
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                ts.append(time.perf_counter() - t0)
            return sorted(ts)[len(ts) // 2]

        t_bf = timed(lambda: EL.load_stacked_experts(idx, pfx, n_experts, out=bf, threads=threads))
        t_q8 = timed(lambda: EL.load_stacked_experts(idx, pfx, n_experts, int8=True, out=q8, threads=threads))

        items = EL.expert_items(idx, pfx, n_experts)
        hdr = {p_: EL.read_header(p_) for p_ in set(idx.values())}
        jobs = sorted((idx[k], hdr[idx[k]][k][2], hdr[idx[k]][k][3] - hdr[idx[k]][k][2], part, slot, hdr[idx[k]][k][1])
                      for k, part, slot in items)
        groups = [jobs[i::ref_threads] for i in range(ref_threads)]  # direct_load.py's default of 8 workers

        def ref_method(int8):
            def work(group):
                st = torch.cuda.Stream()
                with torch.cuda.stream(st):
                    for path, off, n, part, slot, shape in group:
                        fd = os.open(path, os.O_RDONLY)
                        buf = bytearray(n)
                        mv, got = memoryview(buf), 0
                        while got < n:
                            got += os.preadv(fd, [mv[got:]], off + got)
                        os.close(fd)
                        src = torch.frombuffer(buf, dtype=torch.bfloat16).reshape(shape)
                        r0 = inter if part == 1 else 0
                        if int8:
                            qq, ss = fused_moe.quantize_rows_int8(src.to(dev), scale_dtype=torch.bfloat16)
                            qd, sd = (q8["q_d"], q8["s_d"]) if part == 2 else (q8["q_gu"], q8["s_gu"])
                            qd[slot, r0:r0 + qq.shape[0]].copy_(qq)
                            sd[slot, r0:r0 + qq.shape[0]].copy_(ss)
                        else:
                            (bf["w_d"][slot] if part == 2 else bf["w_gu"][slot, r0:r0 + shape[0]]).copy_(src)
                    st.synchronize()
            with ThreadPoolExecutor(ref_threads) as ex:
                list(ex.map(work, groups))

        t_ref_bf = timed(lambda: ref_method(False))
        t_ref_q8 = timed(lambda: ref_method(True))
    pinned = torch.empty(1 << 30, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    t_h2d = timed(lambda: dst.copy_(pinned, non_blocking=True))
    del pinned, dst, bf, q8
    torch.cuda.empty_cache()
    gbs = lambda sec: nbytes / sec / 1e9  # noqa: E731
    return {"file_bytes": nbytes, "threads": threads, "reference_threads": ref_threads, "bf16_s": t_bf, "bf16_GBs": gbs(t_bf), "int8_s": t_q8,
            "int8_GBs": gbs(t_q8), "reference_method_bf16_GBs": gbs(t_ref_bf),
            "reference_method_int8_GBs": gbs(t_ref_q8), "pinned_h2d_GBs": (1 << 30) / t_h2d / 1e9,
            "source": "page cache (files just written)"}


# -------------------------------------------------------------------------------------------- CPU baseline

def cpu_model():
    """The host CPU as /proc/cpuinfo names it: the model name, then family / model / stepping (some hosts report only
    the brand in the name)."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if not ln.strip():
                    break  # the first processor's block
                k, _, v = ln.partition(":")
                fields[k.strip()] = v.strip()
    except OSError:
        return platform.processor() or platform.machine()
    ident = " ".join(f"{k.split()[-1]} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    return f"{fields.get('model name', platform.machine())} ({ident})" if ident else fields.get("model name", "")


def cpu_baseline(b, bias, n=512, warmup=2, reps=7):
    """The reference's CPU torch path for the headline block on all n tokens of the same seeded input: RMSNorm
    and the fp32 router (O.rms_norm, O.router_logits, O.router_select), the per-expert bf16 loop of
    dev/test_moe_prefill.py:24-38 (O.moe_reference_loop: one GEMM pair per active expert, index_add in fp32),
    the residual add. torch's intra-op threads (the box's CPU share); median of `reps` runs after `warmup`."""
    from oracle import moe_oracle as O
    import workloads as W
    cpu = {k: b[k].cpu() for k in ("norm_w", "w32", "w_gu", "w_d")}
    x = W.tokens(n, seed=70, device="cuda").cpu()
    bias_c = bias.cpu()

    def run():
        xn = O.rms_norm(x, cpu["norm_w"], W.EPS)
        ids, wts = O.router_select(O.router_logits(xn, cpu["w32"]), bias_c, scoring="softmax", top_k=W.TOP_K)
        y = O.moe_reference_loop(xn, cpu["w_gu"], cpu["w_d"], ids, wts)
        return (y.to(torch.bfloat16).float() + x.float()).to(torch.bfloat16)

    for _ in range(warmup):
        run()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t)
    t = sorted(ts)[len(ts) // 2]
    return {"value": n / t, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"all {n} tokens of the headline workload: RMSNorm, fp32 router, the reference's per-expert "
                      f"bf16 loop (dev/test_moe_prefill.py:24-38), residual; median of {reps} runs after {warmup} "
                      "warmups",
            "ms_per_step": t * 1e3, "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
            "torch_threads": torch.get_num_threads(), "torch": torch.__version__}


def read_clocks():
    """Current shader and memory clock levels from the amdgpu sysfs tables (the current level is marked '*'); read
    as files, no child process, so the run stays safe under a profiler that initialises the GPU in every process it
    starts."""
    clocks = {}
    for dev in sorted(glob.glob("/sys/class/drm/card*/device")):
        for table in ("pp_dpm_sclk", "pp_dpm_mclk"):
            try:
                with open(os.path.join(dev, table)) as f:
                    cur = [ln.split(":", 1)[-1].strip(" *\n") for ln in f if ln.rstrip().endswith("*")]
            except OSError:
                continue
            if cur:
                clocks[f"{os.path.basename(os.path.dirname(dev))}.{table[7:]}"] = cur[0]
    return clocks or "unavailable"


def box_info():
    """The GPU this run measured (decode timings of one build differ by up to ~35% between boxes). `clocks_idle` is
    read after the work; the headline's `clocks_under_load` is read while its timed replays run."""
    p = torch.cuda.get_device_properties(0)
    return {"name": p.name, "arch": getattr(p, "gcnArchName", ""), "cus": p.multi_processor_count,
            "host": platform.node(), "clocks_idle": read_clocks()}


def main():
    args = parse()
    if args.pmc_probe:
        pmc_probe()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the MoE block path has no multi-GPU code (use --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    import _mingmoe
    import workloads as W
    _mingmoe.load()
    torch.manual_seed(0)
    stream = torch.cuda.Stream()
    t0 = time.time()
    import fused_moe
    b = W.block(seed=0, device="cuda")
    # the prefill layout copies of the gate/up and down stacks, registered for them (load-time, outside the timed
    # region; decode reads w_gu and w_d): every prefill call on these stacks finds them
    fused_moe.prefill_copies(b["w_gu"], b["w_d"])
    bias = W.ragged_bias(device="cuda")
    torch.cuda.synchronize()
    log(f"[bench] block ready {time.time() - t0:.1f}s")
    # A fresh process's first timed work runs about 5 % slower while the GPU clocks ramp up: one untimed pass of the
    # headline first, then the same block on the row layouts the engine stacks (no copies), then the headline.
    prefill_metrics(b, 512, bias, args.steps, args.warmup, stream)
    rows = prefill_metrics(b, 512, bias, args.steps, args.warmup, stream, slabs=False)
    log(f"[bench] prefill 512, row layout: {rows['tokens_per_s']:.0f} tok/s, gate/up {rows['gate_up_us']:.1f} us")
    head = prefill_metrics(b, 512, bias, args.steps, args.warmup, stream)
    log(f"[bench] prefill 512: {head['tokens_per_s']:.0f} tok/s, gate/up {head['gate_up_us']:.1f} us")
    extra = {"prefill_512": head, "prefill_512_row_layout": rows,
             "prefill_512_engine_call": engine_call_metrics(b, 512, bias, stream)}
    log(f"[bench] engine call: {extra['prefill_512_engine_call']}")
    only = set(filter(None, args.only.split(",")))
    want = (lambda k: not args.quick and (not only or k in only))
    if want("zipf"):
        extra["prefill_2048_zipf"] = prefill_metrics(b, 2048, W.zipf_bias(device="cuda"), 10, 2, stream, seed=90)
        log(f"[bench] zipf: {extra['prefill_2048_zipf']}")
    if want("int8"):
        # the headline block with int8 experts and fp32 row scales (the reference's int8 stacks), same masters
        W.quantize_block(b, torch.float32)
        fused_moe.prefill_copies(b["q_gu"], b["q_d"])
        extra["prefill_512_int8_row_layout"] = prefill_metrics(b, 512, bias, 20, 3, stream, int8=True, slabs=False)
        extra["prefill_512_int8"] = prefill_metrics(b, 512, bias, 20, 3, stream, int8=True)
        log(f"[bench] prefill 512 int8: {extra['prefill_512_int8']}")
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(b, bias)
        log(f"[bench] cpu baseline: {cpu}")
    del b
    torch.cuda.empty_cache()
    if want("full") or want("decode") or want("int8"):
        # 28 distinct layers: the full step, and its MoE blocks for the (cold) decode figures
        step = W.ThinkerDecodeStep(28, "cuda")
        torch.cuda.synchronize()
        blocks = [p["blk"] for p in step.L]
        if want("full"):
            extra["full_decode_28l"] = full_decode_metrics(step, stream)
            log(f"[bench] full decode: {extra['full_decode_28l']}")
        if want("decode"):
            extra["decode_bf16_b1"] = decode_metrics(blocks, 1, stream)
            log(f"[bench] decode bf16 b1: {extra['decode_bf16_b1']}")
        if want("int8"):
            for blk in blocks:  # int8 experts with bf16 row scales from the same bf16 masters
                W.quantize_block(blk, torch.bfloat16)
            for n in (1, 2, 4, 8):
                extra[f"decode_int8_b{n}"] = decode_metrics(blocks, n, stream, int8=True)
                log(f"[bench] decode int8 b{n}: {extra[f'decode_int8_b{n}']}")
        del step, blocks
        torch.cuda.empty_cache()
    if want("hybrid"):
        extra["hybrid_decode_28l"] = hybrid_decode_metrics(stream)
        log(f"[bench] hybrid decode: {extra['hybrid_decode_28l']}")
    if want("hybrid") or want("hybrid_prefill"):
        extra["hybrid_prefill_28l"] = hybrid_prefill_metrics(stream)
        log(f"[bench] hybrid prefill: {extra['hybrid_prefill_28l']}")
    if want("talker"):
        torch.cuda.empty_cache()
        extra["talker"] = talker_metrics(stream)
        log(f"[bench] talker: {extra['talker']}")
    if want("ingest"):
        extra["ingest"] = ingest_metrics()
        log(f"[bench] ingest: {extra['ingest']}")
    b_copy_bytes = (W.EXPERTS + 1) * W.expert_bytes()  # both copies: a second gate/up and down stack
    gu_s = head["gate_up_us"] * 1e-6
    achieved = head["gate_up_bytes"] / gu_s / 1e9
    traffic = None
    if not args.no_pmc:
        traffic, detail = pmc_traffic()
        extra["gate_up_traffic"] = dict(detail, algorithmic_bytes=head["gate_up_bytes"])
        log(f"[bench] gate/up traffic: {traffic} ({detail})")
    line = {
        "metric": "MoE layer decode us/token + achieved HBM TB/s; MoE prefill tokens/s + MFMA %",
        "value": head["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "thinker MoE block prefill, 512 tokens, hidden 2048, 64+1 experts x 1408, "
                               "softmax top-6, ragged router bias", "tokens": 512, "hidden": 2048, "experts": 64,
                   "inter": 1408, "top_k": 6, "graph": True,
                   "gate_up_weights": "prefill copy of the gate/up stack (fused_moe.prefill_copies at load, found by "
                                      "the call)",
                   "down_weights": "prefill copy of the down stack (the same)",
                   "copy_bytes_per_layer": b_copy_bytes},
        "roofline": {"bound": "hbm", "kernel": "prefill_gate_up_kernel<false, 128, 8, 64, true>", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": traffic},
        "cpu_baseline": cpu,
        "box": box_info(),
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
