"""Benchmark of the flint attention hot path on one MI355X.

Primary line (`value`): fused decode attention at 32768 cached positions
(benchmark config 3: full layer, f16 KV, 32 q / 4 kv heads, d=128, split-K +
LSE merge + sink). One step = one decode token through 8 full-attention layers,
each with its own 64 MiB KV cache, so a step streams 512 MiB and the 256 MB
Infinity Cache cannot serve it. value = algorithmic KV bytes / step time (GB/s).

Also reported on the same line: decode tok/s at 32k (Flint's 14 full + 35 SWA
layers, attention only), prefill attention TFLOPS at 4000 tokens (config 4,
bf16 KV, full causal and SWA-513), the 16-sequence mixed-context decode
(config 5), the decode kernel's roofline, and the CPU oracle's decode rate on
this host (cpu_baseline; a reported baseline, not the target).

Also on the line: the attention block of a decode step read from a GGUF model (q8_0 q/k/v/o
projections + attention; full layer at 32k and SWA layer), per layer and as tok/s for Flint's
layer mix.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only decode|prefill|config5|blocks]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flint-mac_amd"))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense bf16/f16 MFMA
N_FULL_FLINT, N_SWA_FLINT = 14, 35
# HBM bytes per decode call (attn_decode_kernel + attn_combine_kernel) at 32k, from rocprofv3
# --pmc FETCH_SIZE and WRITE_SIZE runs of `bench.py --only decode --no-cpu`, each scaled by the
# counter's reading for the 64 MiB calibration copy (profiles/decode_32k_f16.md).
DECODE_TRAFFIC_BYTES = 68915950


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


_SLEEP_CYCLES_PER_MS = None


def _sleep_ms(torch, ms):
    """Occupy the current stream for about `ms` ms with torch's bounded clock-spin kernel."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        e0.record()
        torch.cuda._sleep(2_000_000)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = 2_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(ms * _SLEEP_CYCLES_PER_MS))


def queued_launch_ms(torch, step, reps, warmup=2):
    """GPU time per call of `step` (a sequence of library launches on torch's current stream).

    The `reps` calls are enqueued back to back behind a spin kernel that keeps the stream busy
    while the host enqueues them, so the two events bracket the kernels alone (the host's
    per-call cost of Python + ctypes + hipLaunchKernel stays off the GPU timeline) and the
    launches run as an engine issues them: direct dispatches, no graph. Returns
    (ms per call, host-bound flag): the flag is set if the spin ended before the host had
    enqueued every call (then the figure includes host gaps)."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    step()
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) * 1e3
    e_spin, e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    _sleep_ms(torch, min(2.0 * host_ms * reps + 5.0, 2000.0))
    e_spin.record()
    e0.record()
    for _ in range(reps):
        step()
    e1.record()
    host_bound = e_spin.query()  # the spin already finished: the GPU waited for the host
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps, bool(host_bound)


def decode_bytes(n_keys):
    return n_keys * 4 * 128 * 2 * 2  # K and V, f16, 4 kv heads


def prefill_flops(T, window=None):
    keys = sum(min(i + 1, window) if window else i + 1 for i in range(T))
    return 4 * 32 * 128 * keys


def bench_decode_32k(torch, fa, steps, warmup, n_layers=8, ctx=32768):
    import numpy as np
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(2)
    layers = []
    for i in range(n_layers):
        kv = fa.KVLayer(is_swa=False, has_rope=False, n_slots=ctx + 32, kv_dtype="f16",
                        q_norm=rng.uniform(0.5, 1.5, 128), k_norm=rng.uniform(0.5, 1.5, 128),
                        sinks=rng.standard_normal(32), device=dev)
        kv.k.normal_()
        kv.v.normal_()
        layers.append(kv)
    qkv = torch.randn((n_layers, 5120), device=dev)
    att = torch.empty((n_layers, 4096), device=dev)

    def step():
        for i, kv in enumerate(layers):
            kv.decode(qkv[i], att[i], ctx)

    t0 = time.perf_counter()
    ms_per_step, host_bound = queued_launch_ms(torch, step, steps, warmup)
    wall = time.perf_counter() - t0
    avg_launch_ms = ms_per_step / n_layers
    nbytes = decode_bytes(ctx)
    del layers
    torch.cuda.empty_cache()
    return dict(ms_per_step=ms_per_step, avg_launch_ms=avg_launch_ms, bytes_per_launch=nbytes,
                gbs=nbytes * n_layers / (ms_per_step * 1e-3) / 1e9, wall_s=wall, n_layers=n_layers,
                host_bound=host_bound)


def calibration_copy(torch, nbytes=64 << 20):
    """One plain elementwise pass over a known size (reads and writes nbytes): the reference
    point that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def bench_decode_swa(torch, fa, reps=200, pos=32768):
    import numpy as np
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(5)
    n = 8
    layers = [fa.KVLayer(is_swa=True, has_rope=True, kv_dtype="f16", q_norm=rng.uniform(0.5, 1.5, 128),
                         k_norm=rng.uniform(0.5, 1.5, 128), sinks=rng.standard_normal(32), device=dev)
              for _ in range(n)]
    for kv in layers:
        kv.k.normal_()
        kv.v.normal_()
    qkv = torch.randn((n, 5120), device=dev)
    att = torch.empty((n, 4096), device=dev)

    def step():
        for i, kv in enumerate(layers):
            kv.decode(qkv[i], att[i], pos)

    return queued_launch_ms(torch, step, max(1, reps // n))[0] / n


def bench_prefill(torch, fa, T=4000, reps=10):
    import numpy as np
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(3)
    out = {}
    qkv = torch.randn((T, 5120), device=dev)
    att = torch.empty((T, 4096), device=dev)
    for name, is_swa in (("full", False), ("swa", True)):
        kv = fa.KVLayer(is_swa=is_swa, has_rope=is_swa, n_slots=1024 if is_swa else T, kv_dtype="bf16",
                        q_norm=rng.uniform(0.5, 1.5, 128), k_norm=rng.uniform(0.5, 1.5, 128),
                        sinks=rng.standard_normal(32), device=dev)
        for _ in range(2):
            kv.prefill(qkv, att, 0)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            kv.prefill(qkv, att, 0)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        flops = prefill_flops(T, 513 if is_swa else None)
        out[name] = dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12,
                         frac_of_mfma_peak=flops / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS)
    return out


def bench_config5(torch, fa, steps=3):
    """16 sequences, contexts U[4k, 65k] (seed 4), 12 full + 36 SWA layers (1:3), one token per sequence."""
    import numpy as np
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(4)
    n_seq = 16
    ctx = [int(c) for c in rng.integers(4096, 65537, n_seq)]
    cap = (max(ctx) + 1 + 31) // 32 * 32
    pattern = [(i % 4 == 0) for i in range(48)]  # True = full: 12 full, 36 SWA
    layers = []
    for full in pattern:
        kv = fa.KVLayer(is_swa=not full, has_rope=not full, n_slots=cap if full else 1024, kv_dtype="f16",
                        q_norm=rng.uniform(0.5, 1.5, 128), k_norm=rng.uniform(0.5, 1.5, 128),
                        sinks=rng.standard_normal(32), n_seq=n_seq, device=dev)
        kv.k.normal_()
        kv.v.normal_()
        layers.append(kv)
    qkv = torch.randn((n_seq, 5120), device=dev)
    att = torch.empty((n_seq, 4096), device=dev)

    def step():
        for kv in layers:
            kv.decode(qkv, att, ctx)

    ms, _ = queued_launch_ms(torch, step, steps, warmup=1)
    nbytes = sum(12 * decode_bytes(c) + 36 * decode_bytes(min(c, 512)) for c in ctx)
    del layers
    torch.cuda.empty_cache()
    return dict(ms_per_step=ms, tok_s=n_seq / (ms * 1e-3), gbs=nbytes / (ms * 1e-3) / 1e9, contexts=ctx,
                bytes_per_step=nbytes)


def bench_blocks(torch, fa, reps=96, ctx=32768):
    """The attention block of a decode step read from a GGUF file (include/flint_model.h):
    RMSNorm + q/k/v projections, attention, o projection + residual, with q8_0 weights in
    Flint's shapes (random N(0, 1/k) rows, ggml's q8_0 rounding). One full layer at `ctx` cached
    positions and one SWA layer (window 513). The caches hold zeros: the kernels read every byte
    whatever the values. Each block and its attention stage alone are timed like the decode
    line; the projections are the difference."""
    import ctypes
    import tempfile
    import numpy as np
    import gguf_writer as gw
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(6)
    E = 2048

    def q8(n, k):
        return gw.quantize_q8_0((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))

    tensors = [("token_embd.weight", rng.standard_normal((16, E)).astype(np.float32), gw.T_F16),
               ("output_norm.weight", np.ones(E, np.float32), gw.T_F32),
               ("output.weight", np.zeros((1, E), np.float32), gw.T_F16)]
    wbytes = 0
    for il in range(2):
        b = f"blk.{il}."
        tensors.append((b + "attn_norm.weight", rng.uniform(0.5, 1.5, E).astype(np.float32), gw.T_F32))
        for name, n, k in (("attn_q", 4096, E), ("attn_k", 512, E), ("attn_v", 512, E), ("attn_output", E, 4096)):
            rows = q8(n, k)
            wbytes += rows.nbytes if il == 0 else 0
            tensors.append((b + name + ".weight", rows, 8, (k, n)))
        tensors += [(b + "attn_q_norm.weight", rng.uniform(0.5, 1.5, 128).astype(np.float32), gw.T_F32),
                    (b + "attn_k_norm.weight", rng.uniform(0.5, 1.5, 128).astype(np.float32), gw.T_F32),
                    (b + "attn_sinks.weight", rng.standard_normal(32).astype(np.float32), gw.T_F32)]
        tensors += gw.flint_zero_ffn(il)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "blocks.gguf")
        gw.write_gguf(path, gw.flint_meta([0, 1], [0, 1], 513, 1.0e4), tensors)
        model = fa.Model(path, n_ctx=ctx + 32)
    x = torch.randn(E, device=dev) * 0.1
    qkv = torch.randn(5120, device=dev)
    att = torch.empty(4096, device=dev)
    out = {}
    for il, name in ((0, "full"), (1, "swa")):
        desc = model.layer(il)
        t_block = queued_launch_ms(torch, lambda: model.block_decode(il, x, ctx, att), reps)[0]
        t_attn = queued_launch_ms(
            torch, lambda: fa._call(fa.lib().flint_attn_decode, ctypes.byref(desc), fa._ptr(qkv), fa._ptr(att), ctx,
                                    0, ctypes.c_void_p(fa._stream(None))), reps)[0]
        out[name] = dict(block_ms=t_block, attn_ms=t_attn, proj_ms=t_block - t_attn)
    model.close()
    t_proj = 0.5 * (out["full"]["proj_ms"] + out["swa"]["proj_ms"])
    return dict(full_32k_block_ms=out["full"]["block_ms"], swa_block_ms=out["swa"]["block_ms"],
                full_32k_attn_ms=out["full"]["attn_ms"], swa_attn_ms=out["swa"]["attn_ms"],
                proj_ms=t_proj, proj_weight_bytes=wbytes, proj_gbs=wbytes / (t_proj * 1e-3) / 1e9,
                tok_s_32k=1.0 / ((N_FULL_FLINT * out["full"]["block_ms"] + N_SWA_FLINT * out["swa"]["block_ms"])
                                 * 1e-3))


def cpu_baseline(target_s=10.0):
    """The CPU oracle (C restatement of the reference's CPU attention) on this host:
    config-3 decode steps (32768 cached positions, f16-rounded KV)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as fo
    threads = min(os.cpu_count() or 1, 16)
    rng = np.random.default_rng(2)
    n = 32768
    L = fo.Layer(rng.uniform(0.5, 1.5, 128), rng.uniform(0.5, 1.5, 128), rng.standard_normal(32), 0, 0, "f16")
    K = fo.round_store(rng.standard_normal((n + 1, 512)).astype(np.float32), "f16")
    V = fo.round_store(rng.standard_normal((n + 1, 512)).astype(np.float32), "f16")
    qkv = rng.standard_normal(5120).astype(np.float32)
    fo.decode_step(L, qkv, n, K, V, n_threads=threads)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < target_s:
        fo.decode_step(L, qkv, n, K, V, n_threads=threads)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    return dict(value=decode_bytes(n) / dt / 1e9, unit="GB/s", cores=threads, kind="port",
                sample=f"{reps} decode steps of config 3 (32768 cached f16-rounded positions, fp32 scores, "
                       f"double softmax*V) on {threads} threads, {dt * 1e3:.1f} ms/step",
                tok_s_32k_one_layer=1.0 / dt)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["decode", "prefill", "config5", "blocks"], default=None)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU. The attention path would shard by key range (decode, "
              "one LSE merge of per-GPU partials) or by sequence / kv head, but no multi-GPU figure is "
              "measured here. Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import flint_attn as fa
    fa.lib()
    assert torch.cuda.is_available(), "bench needs a GPU"
    res = {}
    if args.only in (None, "decode"):
        log("decode 32k (config 3)")
        res["decode"] = bench_decode_32k(torch, fa, args.steps, args.warmup)
        log(f"decode: {res['decode']}")
        res["swa_ms"] = bench_decode_swa(torch, fa)
        calibration_copy(torch)
        log(f"swa decode per layer: {res['swa_ms']:.4f} ms")
    if args.only in (None, "prefill"):
        log("prefill 4000 (config 4)")
        res["prefill"] = bench_prefill(torch, fa)
        log(f"prefill: {res['prefill']}")
    if args.only in (None, "config5"):
        log("config 5: 16 sequences x 48 layers")
        res["config5"] = bench_config5(torch, fa)
        log(f"config5: ms {res['config5']['ms_per_step']:.3f} tok/s {res['config5']['tok_s']:.1f} "
            f"GB/s {res['config5']['gbs']:.1f}")
    if args.only in (None, "blocks"):
        log("attention blocks from a GGUF model (q8_0 projections)")
        res["blocks"] = bench_blocks(torch, fa)
        log(f"blocks: {res['blocks']}")
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline()
        log(f"cpu: {cpu}")

    line = {
        "metric": "decode attn HBM GB/s + tok/s @32k ctx; prefill attn TFLOPS @4k tokens",
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
    }
    if "decode" in res:
        d = res["decode"]
        t_full = d["avg_launch_ms"]
        t_swa = res["swa_ms"]
        line.update({
            "value": round(d["gbs"], 1),
            "ms_per_step": round(d["ms_per_step"], 5),
            "config": {"workload": "config 3: decode attention, 1 token, full layer, 32768 cached f16 positions, "
                                   "32 q / 4 kv heads, d=128, split-K + LSE merge + sink; step = 8 layers with "
                                   "their own KV (512 MiB streamed per step)",
                       "context": 32768, "layers_per_step": d["n_layers"], "kv_dtype": "f16"},
            "decode_tok_s_32k": round(1.0 / ((N_FULL_FLINT * t_full + N_SWA_FLINT * t_swa) * 1e-3), 1),
            "decode_ms_per_layer_full_32k": round(t_full, 5),
            "decode_ms_per_layer_swa": round(t_swa, 5),
            "roofline": {"bound": "hbm", "achieved": round(d["bytes_per_launch"] / (t_full * 1e-3) / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(d["bytes_per_launch"] / (t_full * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": DECODE_TRAFFIC_BYTES,
                         "kernel": "one flint_attn_decode call = attn_decode_kernel<1, 1> (f16 KV, no V slices; 43 key "
                                   "splits x 4 kv heads = 172 workgroups) + attn_combine_kernel (split merge); "
                                   "time per call from HIP events",
                         "bytes_per_launch": d["bytes_per_launch"], "host_bound": d["host_bound"]},
        })
    if "prefill" in res:
        line["prefill_4000_bf16"] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                                     for k, v in res["prefill"].items()}
    if "config5" in res:
        c = res["config5"]
        line["config5_16seq_48layers"] = {"ms_per_step": round(c["ms_per_step"], 4), "tok_s": round(c["tok_s"], 1),
                                          "gbs": round(c["gbs"], 1), "bytes_per_step": c["bytes_per_step"]}
    if "blocks" in res:
        line["attention_block_decode_q8_0"] = {k: (round(v, 5) if isinstance(v, float) else v)
                                               for k, v in res["blocks"].items()}
    if cpu:
        line["cpu_baseline"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in cpu.items()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
