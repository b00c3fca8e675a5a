"""Benchmark of the flint attention hot path on one MI355X.

Primary line (`value`): fused decode attention at 32768 cached positions
(benchmark config 3: full layer, f16 KV, 32 q / 4 kv heads, d=128, split-K +
LSE merge + sink). One step = one decode token through 8 full-attention layers,
each with its own 64 MiB KV cache, so a step streams 512 MiB and the 256 MB
Infinity Cache cannot serve it. value = algorithmic KV bytes / step time (GB/s).

Also on the same line:
  * a whole decode step of the attention stage at 32k, timed: Flint's 14 full (pos 32768)
    + 35 SWA layers back to back, each with its own cache (decode_step_49_layers_32k);
  * prefill attention at 4000 tokens (config 4, bf16 KV, full causal and SWA-513), with a
    roofline object per layer kind for the larger of its two floors (MFMA on the full layer,
    HBM on the SWA layer, whose fp32 q in and output out outweigh its FLOPs), the other
    fraction beside it;
  * the 16-sequence mixed-context decode (config 5);
  * the attention blocks read from a 49-layer GGUF model (q8_0 q/k/v/o projections +
    attention): one layer of each kind, a whole decode step at 32k, and the layer-major
    prefill of 4000 tokens (flint_attn_model_prefill);
  * the CPU oracle on every core of this host (cpu_baseline; a reported baseline, not the
    target): config-3 decode GB/s and config-4 prefill TFLOPS;
  * what this GPU itself reaches, measured in the same run (measured_limits): a plain 64 MiB
    streaming read, the f16 MFMA rate, and the GPU time of an empty and of a dependent launch.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--only decode|prefill|prefill_full|prefill_swa|config5|model|roofline]
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
# HBM bytes per decode call (attn_decode_kernel + attn_combine_kernel) at 32k, from rocprofv3
# --pmc FETCH_SIZE and WRITE_SIZE runs of `bench.py --only decode --no-cpu`, each scaled by the
# counter's reading for the 64 MiB calibration copy (profiles/decode_32k_f16.md).
DECODE_TRAFFIC_BYTES = 68866200
# HBM bytes per prefill call (kv_prep_kernel + flash_prefill_kernel) at T = 4000, bf16 KV, from
# rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of `bench.py --only prefill_full|prefill_swa
# --no-cpu`, scaled like the decode figure (profiles/prefill_4000_bf16.md); None = not measured.
PREFILL_TRAFFIC_BYTES = {"full": 184807293, "swa": 169446994}
# Flint's 49 layers: full attention (no RoPE) at layers 0, 48 and i % 4 == 1, SWA + RoPE elsewhere
# (/root/reference/src/metal/flint_config.h:37-38): 14 full, 35 SWA
FLINT_FULL_LAYERS = [i == 0 or i == 48 or i % 4 == 1 for i in range(49)]


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
    _sleep_ms(torch, min(4.0 * host_ms * reps + 20.0, 5000.0))
    e_spin.record()
    e0.record()
    for _ in range(reps):
        step()
    e1.record()
    host_bound = e_spin.query()  # the spin already finished: the GPU waited for the host
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps, bool(host_bound)


def bench_roofline(torch):
    """What this GPU itself reaches, measured in the same run with the kernels of
    flint-mac_amd/libflint_probe.so (a measurement library outside the attention library):
      * a plain 64 MiB streaming read (16-byte non-temporal loads, one contiguous range per
        workgroup, two sets of 4, 8 or 12 loads per thread refilled as they are consumed; the
        best is reported) over 8 rotating buffers (512 MiB, beyond the 256 MB Infinity Cache), at
        1024 workgroups and at the config-3 decode's 172;
      * v_mfma_f32_32x32x16_f16 in 4 or 8 independent chains per wave, 8 waves per workgroup
        (two per SIMD), one and four workgroups per CU (the best is reported);
      * the GPU time per launch of an empty kernel, and of a tiny kernel that reads what the
        launch before it wrote (the dependency of a split merge on the kernel before it).
    Each is timed with HIP events around launches queued behind a spin kernel."""
    import ctypes
    path = os.path.join(ROOT, "flint-mac_amd", "libflint_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build with `make -C flint-mac_amd`")
    P = ctypes.CDLL(path)
    vp, i32, u64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint64
    P.flint_probe_stream_read.argtypes = [vp, u64, i32, i32, vp, vp]
    P.flint_probe_mfma.argtypes = [i32, i32, i32, vp, vp]
    P.flint_probe_empty.argtypes = [vp]
    P.flint_probe_chain.argtypes = [vp, vp, vp]
    for f in (P.flint_probe_stream_read, P.flint_probe_mfma, P.flint_probe_empty, P.flint_probe_chain):
        f.restype = i32

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {rc}")

    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nbytes = 64 << 20
    bufs = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(8)]
    sink = torch.zeros(65536, dtype=torch.float32, device="cuda")
    out = {}
    for n_wg in (1024, 172):
        per = nbytes // (16 * n_wg) * 16 * n_wg  # whole 16-byte units per workgroup
        best = None
        for depth in (4, 8, 12):
            it = [0]

            def step(n_wg=n_wg, per=per, depth=depth, it=it):
                b = bufs[it[0] % 8]
                it[0] += 1
                ok(P.flint_probe_stream_read(ctypes.c_void_p(b.data_ptr()), per, n_wg, depth,
                                             ctypes.c_void_p(sink.data_ptr()), stream), "stream read")
            ms, hb = queued_launch_ms(torch, step, 80, warmup=8)
            r = {"us_per_64mib": round(ms * 1e3 * nbytes / per, 3), "gbs": round(per / (ms * 1e-3) / 1e9, 1),
                 "loads_per_set": depth, "host_bound": hb}
            log(f"stream read {n_wg} workgroups: {r}")
            if best is None or r["gbs"] > best["gbs"]:
                best = r
        out[f"stream_read_{n_wg}wg"] = best
    best = None
    # (workgroups, independent chains per wave, iterations): one and four workgroups per CU
    for n_wg, chains, iters in ((256, 4, 2000), (256, 8, 1000), (1024, 4, 500)):
        flops = n_wg * 8 * iters * chains * 32768

        def mstep(n_wg=n_wg, chains=chains, iters=iters):
            ok(P.flint_probe_mfma(n_wg, iters, chains, ctypes.c_void_p(sink.data_ptr()), stream), "mfma")
        ms, hb = queued_launch_ms(torch, mstep, 8, warmup=2)
        r = {"tflops": round(flops / (ms * 1e-3) / 1e12, 1), "ms": round(ms, 4), "workgroups": n_wg,
             "chains_per_wave": chains, "flops_per_launch": flops, "host_bound": hb}
        log(f"mfma: {r}")
        if best is None or r["tflops"] > best["tflops"]:
            best = r
    out["mfma_f16_32x32x16"] = best

    def estep():
        ok(P.flint_probe_empty(stream), "empty")
    ms, hb = queued_launch_ms(torch, estep, 400, warmup=20)
    out["empty_launch_us"] = round(ms * 1e3, 3)
    a = torch.zeros(4096, dtype=torch.float32, device="cuda")
    b = torch.zeros(4096, dtype=torch.float32, device="cuda")
    flip = [0]

    def cstep():
        x, y = (a, b) if flip[0] % 2 == 0 else (b, a)
        flip[0] += 1
        ok(P.flint_probe_chain(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()), stream), "chain")
    ms, hb = queued_launch_ms(torch, cstep, 400, warmup=20)
    out["dependent_launch_us"] = round(ms * 1e3, 3)
    del bufs
    return out


def decode_bytes(n_keys):
    return n_keys * 4 * 128 * 2 * 2  # K and V, f16, 4 kv heads


def prefill_flops(T, window=None):
    keys = sum(min(i + 1, window) if window else i + 1 for i in range(T))
    return 4 * 32 * 128 * keys


def prefill_bytes(T, ring=None, kv_bytes=2):
    """Algorithmic HBM bytes of one prefill call from position 0: the fp32 q|k|v rows read
    (q 4096 + k, v 512 + 512 floats per token), the fp32 attention output written, and the K/V
    rows the cache keeps (all T on a full layer, the last `ring` on an SWA layer) in the cache
    dtype."""
    kept = min(T, ring) if ring else T
    return T * (4096 + 1024) * 4 + T * 4096 * 4 + kept * 1024 * kv_bytes


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


def bench_decode_swa(torch, fa, reps=320, pos=32768):
    """One SWA decode call (513 keys) per layer, cycling through 160 layers' rings (320 MiB, more
    than the 256 MB Infinity Cache), so each call reads its ring from HBM as in a decode step,
    where every layer's ring was last touched a whole step earlier."""
    import numpy as np
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(5)
    n = 160
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


def bench_decode_step_49(torch, fa, steps=6, ctx=32768):
    """A whole decode step of the attention stage at 32k, timed: Flint's 49 layers in order
    (14 full at pos 32768, each with its own 64 MiB cache, and 35 SWA layers with their rings),
    one flint_attn_decode per layer, back to back on one stream (Engine::step's attention
    stages, engine.mm:902-940 / 735-766)."""
    import numpy as np
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(7)
    layers = []
    for full in FLINT_FULL_LAYERS:
        kv = fa.KVLayer(is_swa=not full, has_rope=not full, n_slots=ctx + 32 if full else 1024, kv_dtype="f16",
                        q_norm=rng.uniform(0.5, 1.5, 128), k_norm=rng.uniform(0.5, 1.5, 128),
                        sinks=rng.standard_normal(32), device=dev)
        kv.k.normal_()
        kv.v.normal_()
        layers.append(kv)
    qkv = torch.randn((len(layers), 5120), device=dev)
    att = torch.empty((len(layers), 4096), device=dev)

    def step():
        for i, kv in enumerate(layers):
            kv.decode(qkv[i], att[i], ctx)

    # 6 steps = 378 launches: more queued behind the spin kernel fill the stream's queue, and
    # hipLaunchKernel then blocks until the GPU frees slots, so the host's per-call Python cost
    # (~10 us) would enter the timed region (host_bound)
    ms, host_bound = queued_launch_ms(torch, step, steps, 2)
    nbytes = sum(decode_bytes(ctx) if full else decode_bytes(512) for full in FLINT_FULL_LAYERS)
    del layers
    torch.cuda.empty_cache()
    return dict(ms_per_step=ms, tok_s=1.0 / (ms * 1e-3), gbs=nbytes / (ms * 1e-3) / 1e9, bytes_per_step=nbytes,
                n_full=sum(FLINT_FULL_LAYERS), n_swa=len(FLINT_FULL_LAYERS) - sum(FLINT_FULL_LAYERS),
                host_bound=host_bound)


def bench_prefill(torch, fa, T=4000, reps=10, kinds=("full", "swa")):
    """Config 4: one prefill call of T = 4000 tokens from position 0 (kv_prep_kernel + flash_prefill_kernel),
    bf16 KV, per layer kind; time per call from HIP events around `reps` calls queued behind a spin
    kernel, as the decode line (the events then see the GPU timeline: with the first call launched
    onto an idle GPU right after the start event, the same 10 calls measured 78-80 instead of 71 us
    per SWA call and 151-152 instead of 146-147 us per full-layer call)."""
    import numpy as np
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(3)
    out = {}
    qkv = torch.randn((T, 5120), device=dev)
    att = torch.empty((T, 4096), device=dev)
    for name in kinds:
        is_swa = name == "swa"
        kv = fa.KVLayer(is_swa=is_swa, has_rope=is_swa, n_slots=1024 if is_swa else T, kv_dtype="bf16",
                        q_norm=rng.uniform(0.5, 1.5, 128), k_norm=rng.uniform(0.5, 1.5, 128),
                        sinks=rng.standard_normal(32), device=dev)
        ms, host_bound = queued_launch_ms(torch, lambda: kv.prefill(qkv, att, 0), reps)
        flops = prefill_flops(T, 513 if is_swa else None)
        nbytes = prefill_bytes(T, 1024 if is_swa else None)
        tflops = flops / (ms * 1e-3) / 1e12
        gbs = nbytes / (ms * 1e-3) / 1e9
        # the call's two floors at the published peaks; the roofline object is the one of the larger
        # floor (MFMA on a full causal layer, HBM on an SWA-513 layer), with the other fraction beside it
        floor_us = {"mfma": flops / (MFMA_PEAK_TFLOPS * 1e12) * 1e6, "hbm": nbytes / (HBM_PEAK_GBS * 1e9) * 1e6}
        mfma_frac, hbm_frac = tflops / MFMA_PEAK_TFLOPS, gbs / HBM_PEAK_GBS
        kernel = ("one flint_attn_prefill call on a " + ("SWA-513" if is_swa else "full causal")
                  + " layer = kv_prep_kernel + flash_prefill_kernel (f16 MFMA 32x32x16 on the exact f16 copy of "
                  "the bf16 K/V); achieved = algorithmic FLOPs or bytes / time per call from HIP events around "
                  "calls queued behind a spin kernel")
        if floor_us["mfma"] >= floor_us["hbm"]:
            roof = {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(mfma_frac, 4), "hbm_frac": round(hbm_frac, 4)}
        else:
            roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(hbm_frac, 4), "mfma_frac": round(mfma_frac, 4)}
        roof.update({"traffic": PREFILL_TRAFFIC_BYTES[name], "bytes_per_launch": nbytes, "flops_per_launch": flops,
                     "floor_us": {k: round(v, 2) for k, v in floor_us.items()}, "kernel": kernel})
        out[name] = dict(ms=ms, flops=flops, tflops=tflops, frac_of_mfma_peak=mfma_frac, gbs=gbs,
                         frac_of_hbm_peak=hbm_frac, host_bound=host_bound, roofline=roof)
        del kv
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


def bench_model(torch, fa, reps=48, ctx=32768, T_prefill=4000):
    """The attention blocks of a 49-layer Flint GGUF (include/flint_model.h): RMSNorm + q/k/v
    projections, attention, o projection + residual, with q8_0 weights in Flint's shapes (random
    N(0, 1/k) rows with ggml's q8_0 rounding; one set of rows written into every layer, each layer
    its own copy in HBM) and Flint's layer pattern. The caches hold zeros: the kernels read every
    byte whatever the values.
      * the full layers' blocks at `ctx` cached positions and the SWA layers' blocks, each block
        and its attention stage alone timed like the decode line, each call on the next layer of
        its kind (the projections are the difference);
      * flint_attn_model_prefill of T_prefill tokens from position 0 (embedding, then layer-major
        blocks), and of the whole ctx-token prompt;
      * then flint_attn_model_step (Engine::step over the blocks) at position ctx: 8 tokens per
        rep, rolled back to ctx between reps."""
    import ctypes
    import tempfile
    import numpy as np
    import gguf_writer as gw
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(6)
    E = 2048

    def q8(n, k):
        return gw.quantize_q8_0((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))

    rows = {name: (q8(n, k), (k, n)) for name, n, k in
            (("attn_q", 4096, E), ("attn_k", 512, E), ("attn_v", 512, E), ("attn_output", E, 4096))}
    wbytes = sum(r.nbytes for r, _ in rows.values())
    n_vocab = 1024
    tensors = [("token_embd.weight", rng.standard_normal((n_vocab, E)).astype(np.float32), gw.T_F16),
               ("output_norm.weight", np.ones(E, np.float32), gw.T_F32),
               ("output.weight", np.zeros((1, E), np.float32), gw.T_F16)]
    for il in range(len(FLINT_FULL_LAYERS)):
        b = f"blk.{il}."
        tensors.append((b + "attn_norm.weight", rng.uniform(0.5, 1.5, E).astype(np.float32), gw.T_F32))
        for name, (r, dims) in rows.items():
            tensors.append((b + name + ".weight", r, 8, dims))
        tensors += [(b + "attn_q_norm.weight", rng.uniform(0.5, 1.5, 128).astype(np.float32), gw.T_F32),
                    (b + "attn_k_norm.weight", rng.uniform(0.5, 1.5, 128).astype(np.float32), gw.T_F32),
                    (b + "attn_sinks.weight", rng.standard_normal(32).astype(np.float32), gw.T_F32)]
        tensors += gw.flint_zero_ffn(il)
    is_swa = [not f for f in FLINT_FULL_LAYERS]
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "flint49.gguf")
        gw.write_gguf(path, gw.flint_meta(is_swa, is_swa, 513, 1.0e4), tensors)
        del tensors
        model = fa.Model(path, n_ctx=ctx + 64)
    x = torch.randn(E, device=dev) * 0.1
    qkv = torch.randn(5120, device=dev)
    att = torch.empty(4096, device=dev)
    out = {}
    # Each call takes the next layer of the kind, so every call reads weights and a cache that
    # the calls before it did not leave in the GPU's caches (one layer's 20 MB of projection
    # weights fits in the 256 MB Infinity Cache and would be served from there if repeated),
    # as in a step through the model.
    for kind_full, name in ((True, "full"), (False, "swa")):
        ils = [il for il, f in enumerate(FLINT_FULL_LAYERS) if f == kind_full]
        descs = [model.layer(il) for il in ils]
        nxt = [0]

        def block():
            i = nxt[0] = (nxt[0] + 1) % len(ils)
            model.block_decode(ils[i], x, ctx, att)

        def attn():
            i = nxt[0] = (nxt[0] + 1) % len(ils)
            fa._call(fa.lib().flint_attn_decode, ctypes.byref(descs[i]), fa._ptr(qkv), fa._ptr(att), ctx, 0,
                     ctypes.c_void_p(fa._stream(None)))
        t_block = queued_launch_ms(torch, block, reps)[0]
        t_attn = queued_launch_ms(torch, attn, reps)[0]
        out[name] = dict(block_ms=t_block, attn_ms=t_attn, proj_ms=t_block - t_attn)
    t_proj = 0.5 * (out["full"]["proj_ms"] + out["swa"]["proj_ms"])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, reps):
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    # layer-major prefill (flint_attn_model_prefill: embedding, then every layer's block over the
    # whole prompt) of T_prefill tokens from position 0
    tokens = [int(t) for t in rng.integers(0, n_vocab, ctx)]
    X = torch.empty((ctx, E), device=dev)

    def prefill_from_0(n):
        model.truncate(0)
        model.prefill(tokens[:n], X[:n])

    prefill_from_0(T_prefill)  # warm-up (workspace growth)
    t_prefill = timed(lambda: prefill_from_0(T_prefill), 2)
    # the whole 32k prompt, then Engine::step at position ctx (flint_attn_model_step: the token's
    # embedding and the 49 blocks, one C call per token); each rep steps 8 tokens from ctx
    t_prefill_ctx = timed(lambda: prefill_from_0(ctx), 1)
    xs = torch.empty((8, E), device=dev)

    def eight_steps():
        model.truncate(ctx)
        for i in range(8):
            model.step(17 + i, xs[i])

    eight_steps()
    t_step = timed(eight_steps, 3) / 8
    # one profiled step (flint_attn_model_enable_profiling / _last_profile): GPU time per kind of
    # stage, summed over the 49 layers (the marks between stages add a little to the total)
    model.truncate(ctx)
    model.enable_profiling(True)
    model.step(17, xs[0])
    shares = {}
    for label, ms in model.last_profile():
        kind = label.rsplit(".", 1)[-1]
        shares[kind] = shares.get(kind, 0.0) + ms
    profiled_step_ms = model.last_gpu_ms()
    model.enable_profiling(False)
    model.close()
    return dict(full_32k_block_ms=out["full"]["block_ms"], swa_block_ms=out["swa"]["block_ms"],
                full_32k_attn_ms=out["full"]["attn_ms"], swa_attn_ms=out["swa"]["attn_ms"],
                proj_ms=t_proj, proj_weight_bytes=wbytes, proj_gbs=wbytes / (t_proj * 1e-3) / 1e9,
                step_32k_ms=t_step, step_tok_s_32k=1.0 / (t_step * 1e-3),
                step_profile_ms={k: round(v, 5) for k, v in shares.items()},
                step_profiled_ms=profiled_step_ms,
                prefill_4000_ms=t_prefill, prefill_4000_tok_s=T_prefill / (t_prefill * 1e-3),
                prefill_32k_ms=t_prefill_ctx, prefill_32k_tok_s=ctx / (t_prefill_ctx * 1e-3))


def cpu_baseline(decode_s=10.0, prefill_s=6.0):
    """The CPU oracle (C restatement of the reference's CPU attention, ref_model.cpp:95-149) on every
    core this process may use: config-3 decode steps (32768 cached f16-rounded positions; threads over
    the 32 q heads, so at most 32) and config-4 prefill (T = 4000, bf16-rounded KV; (row, head) pairs
    over all cores) on a sample of rows, full causal and SWA-513, as TFLOPS over the sample's
    algorithmic FLOPs."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as fo
    cores = len(os.sched_getaffinity(0))
    dthreads = min(cores, 32)
    rng = np.random.default_rng(2)
    n = 32768
    L = fo.Layer(rng.uniform(0.5, 1.5, 128), rng.uniform(0.5, 1.5, 128), rng.standard_normal(32), 0, 0, "f16")
    K = fo.round_store(rng.standard_normal((n + 1, 512)).astype(np.float32), "f16")
    V = fo.round_store(rng.standard_normal((n + 1, 512)).astype(np.float32), "f16")
    qkv = rng.standard_normal(5120).astype(np.float32)
    fo.decode_step(L, qkv, n, K, V, n_threads=dthreads)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < decode_s:
        fo.decode_step(L, qkv, n, K, V, n_threads=dthreads)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    del K, V
    # config 4: sample rows at the end of the prompt (the longest key ranges of the full layer)
    T = 4000
    rng = np.random.default_rng(3)
    qkv4 = rng.standard_normal((T, 5120)).astype(np.float32)
    pre = {}
    for name, is_swa in (("full", 0), ("swa", 1)):
        Lp = fo.Layer(rng.uniform(0.5, 1.5, 128), rng.uniform(0.5, 1.5, 128), rng.standard_normal(32), is_swa, is_swa,
                      "bf16", 1e4)
        Kp = np.zeros((T, 512), np.float32)
        Vp = np.zeros((T, 512), np.float32)
        # q/k/v of all 4000 tokens alone (no rows), then 64 rows to calibrate, then a sample of rows
        # sized to ~prefill_s seconds; the sample is charged its share (rows / T) of the q/k/v time
        r1 = T
        t0 = time.perf_counter()
        fo.prefill_rows(Lp, qkv4, 0, Kp, Vp, r1, r1, n_threads=cores)
        t_prep = time.perf_counter() - t0
        t0 = time.perf_counter()
        fo.prefill_rows(Lp, qkv4, 0, Kp, Vp, r1 - 64, r1, n_threads=cores)
        per_row = max(time.perf_counter() - t0 - t_prep, 1e-6) / 64
        rows = int(min(T, max(64, prefill_s / per_row)))
        t0 = time.perf_counter()
        fo.prefill_rows(Lp, qkv4, 0, Kp, Vp, r1 - rows, r1, n_threads=cores)
        dtp = max(time.perf_counter() - t0 - t_prep, 1e-6) + t_prep * rows / T
        keys = sum(min(i + 1, 513) if is_swa else i + 1 for i in range(r1 - rows, r1))
        flops = 4 * 32 * 128 * keys
        pre[name] = dict(tflops=flops / dtp / 1e12, rows=rows, seconds=dtp)
    return dict(value=decode_bytes(n) / dt / 1e9, unit="GB/s", cores=cores, kind="port",
                sample=f"config 3: {reps} decode steps (32768 cached f16-rounded positions, fp32 scores, double "
                       f"softmax*V) on {dthreads} threads (one per q head at most), {dt * 1e3:.1f} ms/step; config 4: "
                       f"the last {pre['full']['rows']} (full) / {pre['swa']['rows']} (SWA) of 4000 prefill rows "
                       f"on {cores} threads, charged their share of the 4000 tokens' q/k/v prep",
                decode_threads=dthreads, tok_s_32k_one_layer=1.0 / dt,
                prefill_4000_full_tflops=pre["full"]["tflops"], prefill_4000_swa_tflops=pre["swa"]["tflops"])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["decode", "prefill", "prefill_full", "prefill_swa", "config5", "model",
                                       "roofline"], default=None)
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
    if args.only in (None, "roofline"):
        log("measured limits of this GPU (libflint_probe.so)")
        res["roofline"] = bench_roofline(torch)
        log(f"measured: {res['roofline']}")
    if args.only in (None, "decode"):
        log("decode 32k (config 3)")
        res["decode"] = bench_decode_32k(torch, fa, args.steps, args.warmup)
        log(f"decode: {res['decode']}")
        res["swa_ms"] = bench_decode_swa(torch, fa)
        log(f"swa decode per layer: {res['swa_ms']:.4f} ms")
        res["step49"] = bench_decode_step_49(torch, fa)
        log(f"decode step, 49 layers at 32k: {res['step49']}")
        calibration_copy(torch)
    if args.only in (None, "prefill", "prefill_full", "prefill_swa"):
        kinds = {"prefill_full": ("full",), "prefill_swa": ("swa",)}.get(args.only, ("full", "swa"))
        log(f"prefill 4000 (config 4): {kinds}")
        res["prefill"] = bench_prefill(torch, fa, kinds=kinds)
        log(f"prefill: {res['prefill']}")
        calibration_copy(torch)
    if args.only in (None, "config5"):
        log("config 5: 16 sequences x 48 layers")
        res["config5"] = bench_config5(torch, fa)
        log(f"config5: ms {res['config5']['ms_per_step']:.3f} tok/s {res['config5']['tok_s']:.1f} "
            f"GB/s {res['config5']['gbs']:.1f}")
    if args.only in (None, "model"):
        log("attention blocks of a 49-layer GGUF model (q8_0 projections)")
        res["model"] = bench_model(torch, fa)
        log(f"model: {res['model']}")
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
        s49 = res["step49"]
        line.update({
            "value": round(d["gbs"], 1),
            "ms_per_step": round(d["ms_per_step"], 5),
            "config": {"workload": "config 3: decode attention, 1 token, full layer, 32768 cached f16 positions, "
                                   "32 q / 4 kv heads, d=128, split-K + LSE merge + sink; step = 8 layers with "
                                   "their own KV (512 MiB streamed per step)",
                       "context": 32768, "layers_per_step": d["n_layers"], "kv_dtype": "f16"},
            "decode_tok_s_32k": round(s49["tok_s"], 1),
            "decode_step_49_layers_32k": {"ms": round(s49["ms_per_step"], 5), "tok_s": round(s49["tok_s"], 1),
                                          "gbs": round(s49["gbs"], 1), "bytes_per_step": s49["bytes_per_step"],
                                          "layers": f"{s49['n_full']} full (pos 32768) + {s49['n_swa']} SWA, "
                                                    "flint_config.h:37-38 order, one flint_attn_decode each, timed "
                                                    "as one sequence", "host_bound": s49["host_bound"]},
            "decode_ms_per_layer_full_32k": round(t_full, 5),
            "decode_ms_per_layer_swa": round(t_swa, 5),
            "roofline": {"bound": "hbm", "achieved": round(d["bytes_per_launch"] / (t_full * 1e-3) / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(d["bytes_per_launch"] / (t_full * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": DECODE_TRAFFIC_BYTES,
                         "kernel": "one flint_attn_decode call = attn_decode_kernel<1, 1> (f16 KV, no V slices; 43 key "
                                   "splits x 4 kv heads = 172 workgroups) + attn_combine_kernel (split merge, 32 workgroups of 4 waves, one lane per split); "
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
    if "roofline" in res:
        line["measured_limits"] = res["roofline"]
    if "model" in res:
        line["attention_blocks_q8_0_49_layers"] = {k: (round(v, 5) if isinstance(v, float) else v)
                                                   for k, v in res["model"].items()}
    if cpu:
        line["cpu_baseline"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in cpu.items()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
