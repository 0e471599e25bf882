"""KIVI hot-path benchmark on one MI355X.

Headline (``value``): packed-KV decode throughput at benchmark config 4
(Llama-3-8B GQA shape: B=64, 32 q heads / 8 kv heads, D=128, context 8192,
R=128, G=32).  One step = the fused packed decode attention for one query
token per sequence, which also files the step's new K/V into the HBM
residual ring, then a flush of the 32 oldest residual tokens into the packed
store whenever the window reaches R.  ``value`` is algorithmic bytes moved by
those steps / GPU time of the K timed steps, in GB/s.  The first timed step
is a flush step, so K steps hold ceil(K / 32) flushes (reported).

Also reported: the attention kernel alone against the 8 TB/s HBM roofline
(``roofline``: context 8192 = 8064 quantised + a full window of 128; HBM
traffic from two rocprofv3 counter passes in the same run), configs 3 and 5
at their stated token counts, the config-2 codec ops through ``_C``
(quantise, dequantise, round-trip), the batched prefill flush, greedy
decoding end to end (GPT-2 as the reference times it; a Llama-3-8B-shaped
model at serving scale), and CPU baselines of the reference path timed on
the host over the same K/V bits.

Algorithmic bytes (per (batch, kv-head)):
  attention : D*Tq/4 + 8*D*Tq/Gk + Tq*D/4 + 8*Tq*D/Gv + 2*r*Tr*D + 8*(Hq/Hkv)*D
              (r = 4 for the fp32 ring, 2 for the bf16 ring of the
              ``attention_config4_ring_bf16`` leg; the step's new token is
              read as part of Tr)
  append    : 4*D*2 written (the new token's K and V into the ring)
  flush     : 8*G*D (read residual) + G*D/4 + 8*D + G*D/4 + 8*G*D/Gv (write)
  quantise  : per tensor of N fp32: 4N read + N/4 + 8N/G written
  dequantise: per tensor: N/4 + 8N/G read + 4N written
  round-trip: per tensor: 4N read + 4N written
"""

from __future__ import annotations

import argparse
import contextlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def attn_bytes(B, Hq, Hkv, D, Tq, Tr, Gk, Gv, ring_bytes=4):
    """Algorithmic bytes of one decode-attention call: codes, scales and zeros
    of Tq quantised tokens, Tr residual tokens of K and V (ring_bytes per
    element: 4 fp32, 2 bf16/fp16), q and o (fp32)."""
    per = (D * Tq // 4 + 8 * D * Tq // Gk + Tq * D // 4 + 8 * Tq * D // Gv
           + 2 * ring_bytes * Tr * D + 8 * (Hq // Hkv) * D)
    return per * B * Hkv


def flush_bytes(B, Hkv, D, G, Gv):
    return B * Hkv * (8 * G * D + G * D // 4 + 8 * D + G * D // 4 + 8 * G * D // Gv)


def fused_append_bytes(B, Hkv, D):
    return B * Hkv * 8 * D


def quant_bytes(N, G):
    return 4 * N + N // 4 + 8 * N // G


def dequant_bytes(N, G):
    return N // 4 + 8 * N // G + 4 * N


def roundtrip_bytes(N):
    return 8 * N


# --------------------------------------------------------------------------
# GPU workloads
# --------------------------------------------------------------------------
def synth_kv(B, H, T, D, seed):
    """Seeded synthetic K/V ``[B, H, T, D]`` fp32, made on the CPU (so that
    the GPU runs, the CPU baseline and the parity tests see identical bits):
    N(0,1); keys with 4 fixed channels per kv head x10 (channel outliers);
    values with round(2% of T) token positions per (b, kv head) x8 (token
    outliers)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, H, T, D, generator=g)
    v = torch.randn(B, H, T, D, generator=g)
    for h in range(H):
        ch = torch.randperm(D, generator=g)[:min(4, D)]
        k[:, h, :, ch] *= 10.0
    n = max(1, round(0.02 * T))
    for b in range(B):
        for h in range(H):
            tok = torch.randperm(T, generator=g)[:n]
            v[b, h, tok] *= 8.0
    return k, v


def store_tokens(Tq, Tr, G, R):
    """Tokens to feed an empty store through ``extend(flush_at=R)`` (the
    KiviCache rule: flush the G oldest while the residual holds >= R) so
    that it ends with Tq quantised and Tr residual tokens; Tr must lie in
    [R - G, R - 1] (what that rule leaves) and Tq be a multiple of G."""
    if Tq % G or not R - G <= Tr < R:
        raise ValueError(f"Tq={Tq}, Tr={Tr} is not a state extend(flush_at={R}) leaves")
    return Tq + Tr


def make_store(k, v, G, Gv, R, device, extra_chunks=16):
    """A PackedKVStore fed with CPU K/V ``[B, Hkv, T, D]`` by one batched
    ``extend`` (one flush launch for every chunk owed, then the residual
    copy), as a prompt would be."""
    from intel_kivi_hybrid_amd.store import PackedKVStore
    B, Hkv, T, D = k.shape
    st = PackedKVStore(B, Hkv, D, G, R, device, group_size_v=Gv,
                       chunk_capacity=T // G + extra_chunks)
    st.extend(k.to(device), v.to(device), flush_at=R)
    return st


def settle_clocks(fn, seconds=0.1, min_calls=20):
    """Runs fn back to back for ~`seconds` of GPU time (untimed).  From idle,
    MI355X clocks take tens of milliseconds to ramp up (and dip once on the
    way): timing without this reports the first calls ~20% slow."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while n < min_calls or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
        if n % 10 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_calls(fn, iters, blocks=5):
    """Average GPU time of one ``fn()`` call, in microseconds.  HIP events on
    torch's current stream (the stream every launch here goes to) bracket
    blocks of back-to-back calls: the host issues a call in a fraction of its
    GPU time, so the queue never drains, and a block's time per call is the
    kernels' duration plus the launch gaps, without host latency.  An
    untimed call ahead of each block keeps the GPU busy while the block's
    first call is issued (otherwise the start event would also time the
    host's issue of that call)."""
    import torch
    settle_clocks(fn)
    per_block = max(1, iters // blocks)
    ms = []
    for _ in range(blocks):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        fn()
        e0.record()
        for _ in range(per_block):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1) / per_block)
    ms.sort()
    return {"avg_us": 1e3 * sum(ms) / len(ms), "median_us": 1e3 * ms[len(ms) // 2]}


def time_attention(st, q, iters, rotate=None):
    """One fused-attention call over the store as it stands.  ``rotate``: more
    stores of the same shape, called in turn with ``st`` so that the bytes
    touched between two calls on one store exceed the 256 MB MALL."""
    import torch
    out = torch.empty_like(q)
    stores = [st] + list(rotate or [])
    turn = [0]

    def call():
        stores[turn[0]].attention(q, out=out)
        turn[0] = (turn[0] + 1) % len(stores)
    r = time_calls(call, iters)
    Hq = q.shape[1]
    nbytes = attn_bytes(st.B, Hq, st.H, st.D, st.quantized_tokens, st.res_len, st.G, st.Gv,
                        st.k_res.element_size())
    ws = st.workspace_bytes(Hq)
    r.update({"bytes": nbytes, "gbs": nbytes / (r["avg_us"] * 1e-6) / 1e9,
              "Tq": st.quantized_tokens, "Tr": st.res_len,
              "splits": ws // (st.B * Hq * (st.D + 2) * 4) if ws else 1})
    return r


def time_flush(st, iters=50):
    """One decode-time flush (the G oldest residual tokens of every (b, kv
    head) into a new chunk).  A flush moves no ring data, so undoing its
    bookkeeping re-arms the same flush; the store is left as it was."""
    if st.res_len < st.G:
        raise ValueError("time_flush needs a window of at least G tokens")
    st.reserve(st.n_chunks + 1)

    def one():
        st.flush()
        st.n_chunks -= 1
        st.res_start = (st.res_start - st.G) % st.R
        st.res_len += st.G

    r = time_calls(one, iters)
    nbytes = flush_bytes(st.B, st.H, st.D, st.G, st.Gv)
    r.update({"bytes": nbytes, "gbs": nbytes / (r["avg_us"] * 1e-6) / 1e9})
    return r


def decode_loop(st, q_all, k_new, v_new, steps, warmup, R):
    """The timed decode loop.  Step i: the new token is staged (the attention
    launch writes it into the ring itself), the fused attention runs for one
    query token per sequence, and the G oldest residual tokens are quantised
    once the window holds R.  The caller sets the store up so that the first
    timed step is a flush step: K timed steps then hold ceil(K / G) flushes
    (exactly K / G when G divides K)."""
    import torch
    B, Hkv, D, G, Gv = st.B, st.H, st.D, st.G, st.Gv
    Hq = q_all.shape[2]
    out = torch.empty(B, Hq, D, device=q_all.device)

    def step(i):
        st.stage_token(k_new[:, :, i:i + 1], v_new[:, :, i:i + 1])
        nb = attn_bytes(B, Hq, Hkv, D, st.quantized_tokens, st.res_len, G, Gv)
        nb += fused_append_bytes(B, Hkv, D)
        st.attention(q_all[i], out=out)
        flushes = 0
        while st.res_len >= R:
            st.flush()
            flushes += 1
        nb += flushes * flush_bytes(B, Hkv, D, G, Gv)
        return nb, flushes

    settle_clocks(lambda: st.attention(q_all[0], out=out))
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    total_bytes = total_flushes = 0
    ctx0 = st.quantized_tokens + st.res_len + 1
    wall0 = time.perf_counter()
    t0.record()
    for i in range(warmup, warmup + steps):
        nb, fl = step(i)
        total_bytes += nb
        total_flushes += fl
    t1.record()
    submit = time.perf_counter() - wall0     # host time to issue the K steps
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1)
    return {"ms": ms, "submit_s": submit, "bytes": total_bytes, "flushes": total_flushes,
            "context": [ctx0, st.quantized_tokens + st.res_len],
            "gbs": total_bytes / (ms * 1e-3) / 1e9, "ms_per_step": ms / steps}


def codec_bench(kt, v, G, iters=50):
    """Config 2 through the ``_C`` ops on device-resident inputs: keys
    ``kt [B,H,D,Seq]`` quantised per channel along tokens, values
    ``v [B,H,Seq,D]`` per token along channels, both in groups of G.  Times
    the K+V pair of each op the reference exposes: quantise, dequantise and
    the fused round-trip (the op KiviCache's flush calls,
    src/kivi_sycl/cache/manager.py:338,345).  Mtokens/s counts (b, t)
    positions with all heads of K and V."""
    import torch
    from intel_kivi_hybrid_amd import _C
    B, H, D, S = kt.shape
    N = kt.numel()
    kp = torch.empty(N // 4, dtype=torch.uint8, device=kt.device)
    ks = torch.empty(N // G, device=kt.device)
    kz = torch.empty(N // G, device=kt.device)
    vp, vs, vz = torch.empty_like(kp), torch.empty_like(ks), torch.empty_like(kz)
    kd = torch.empty_like(kt)
    vd = torch.empty_like(v)

    def quant():
        _C.quantize_keys_async(kt, kp, ks, kz, G)
        _C.quantize_values_async(v, vp, vs, vz, D, G)

    def dequant():
        _C.dequantize_keys_async(kp, ks, kz, kd, G)
        _C.dequantize_values_async(vp, vs, vz, vd, D, G)

    def roundtrip():
        _C.quant_dequant_roundtrip_keys_async(kt, kd, G)
        _C.quant_dequant_roundtrip_values_async(v, vd, D, G)

    tokens = B * S
    algo = {"quantize": 2 * quant_bytes(N, G), "dequantize": 2 * dequant_bytes(N, G),
            "roundtrip": 2 * roundtrip_bytes(N)}
    res = {}
    for name, fn in (("quantize", quant), ("dequantize", dequant), ("roundtrip", roundtrip)):
        r = time_calls(fn, iters)
        us = r["avg_us"]
        res[name] = {"us_per_pair": round(us, 1), "gbs": round(algo[name] / (us * 1e-6) / 1e9, 1),
                     "mtokens_s": round(tokens / us, 2), "bytes": algo[name]}
    # round-trip error / scale (reported, not gated)
    _C.quant_dequant_roundtrip_values(v, vd, D, G)
    _C.quantize_values(v, vp, vs, vz, D, G)
    err = (vd - v).abs().reshape(-1, G).amax(dim=1)
    res["max_err_over_scale"] = float((err / vs).max())
    return res


def prefill_bench(k, v, device, iters=20):
    """Batched prefill: a prompt ``k``/``v [B, H, T, D]`` appended to an
    empty PackedKVStore (R=128, G=32), which quantises every chunk it owes in
    one launch reading the K/V in place and copies the leftover tokens into
    its residual ring (of the prompt's type, as KiviPackedCache keeps it);
    fp32 and bf16 inputs.  Algorithmic bytes: the flushed tokens' K/V read
    once plus the codes, scales and zeros written, and the leftover tokens
    read and written once; Mtokens/s counts (b, t) positions with all heads
    of K and V."""
    import torch
    from intel_kivi_hybrid_amd.store import PackedKVStore
    B, H, T, D = k.shape
    G, R = 32, 128
    out = {}
    for name, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        kk, vv = k.to(device, dt), v.to(device, dt)
        st = PackedKVStore(B, H, D, G, R, device, chunk_capacity=T // G + 1, residual_dtype=dt)

        def one():
            st.reset()
            st.extend(kk, vv, flush_at=R)

        us = time_calls(one, iters)["avg_us"]
        n_tok = st.n_chunks * G
        nbytes = (2 * B * H * n_tok * D * kk.element_size()       # K/V read
                  + 2 * B * H * n_tok * D // 4                     # codes
                  + B * H * st.n_chunks * D * 8                    # key scales + zeros
                  + B * H * n_tok * (D // G) * 8                   # value scales + zeros
                  + 2 * B * H * st.res_len * D * 2 * kk.element_size())   # leftover tokens
        out[name] = {"us": round(us, 1), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "mtokens_s": round(B * n_tok / us, 1), "chunks": st.n_chunks,
                     "bytes": nbytes}
        del st, kk, vv
    return out


# --------------------------------------------------------------------------
# HBM traffic of the headline kernel (rocprofv3 counters, measured in the run)
# --------------------------------------------------------------------------
ATTN_KERNEL = "attn_mfma_kernel"
COPY_BYTES = 512 << 20


def traffic_workload(dev):
    """Child-process workload for the counter passes: a 512 MiB device copy
    (calibration: it reads and writes COPY_BYTES) and the config-4 attention
    at the roofline state.  Counters do not depend on the values, so the
    store is filled from the GPU's own generator here (fast)."""
    import torch
    from intel_kivi_hybrid_amd.store import PackedKVStore
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(7)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    del src, dst
    B, Hq, Hkv, D, T, R, G = CONFIG4
    g = torch.Generator(device=dev).manual_seed(11)
    st = PackedKVStore(B, Hkv, D, G, R, dev, chunk_capacity=T // G + 1)
    st.extend(torch.randn(B, Hkv, T - 1, D, generator=g, device=dev),
              torch.randn(B, Hkv, T - 1, D, generator=g, device=dev), flush_at=R)
    st.append(torch.randn(B, Hkv, 1, D, generator=g, device=dev),
              torch.randn(B, Hkv, 1, D, generator=g, device=dev))
    q = torch.randn(B, Hq, D, generator=g, device=dev) * D ** -0.5
    for _ in range(3):
        st.attention(q)
    torch.cuda.synchronize()


def _counter_means(outdir, counter):
    """Mean value of ``counter`` per dispatch for the copy kernel and the
    attention kernel, from rocprofv3's counter-collection CSV."""
    import csv
    import glob
    vals = {"copy": [], "attn": []}
    for path in glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                name = row.get("Kernel_Name", "")
                key = "attn" if ATTN_KERNEL in name else "copy" if "copyBuffer" in name else None
                if key:
                    vals[key].append(float(row["Counter_Value"]))
    if not vals["copy"] or not vals["attn"]:
        raise RuntimeError(f"no {counter} rows for the copy and attention kernels in {outdir}")
    return {k: sum(v) / len(v) for k, v in vals.items()}


def measure_traffic(algo_bytes, log):
    """HBM bytes per config-4 attention launch from two rocprofv3 --pmc passes
    (FETCH_SIZE, then WRITE_SIZE, in KiB per dispatch) over a child process
    running traffic_workload(), each scaled by what the counter reads for the
    512 MiB copy in the same pass.  Returns the roofline's traffic fields, or
    null traffic with the reason when the profiler is unavailable."""
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return {"traffic": None, "traffic_note": "rocprofv3 not found"}
    means = {}
    try:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            outdir = tempfile.mkdtemp(prefix=f"kivi_pmc_{counter}_")
            cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", outdir, "-o", "p",
                   "--", sys.executable, os.path.abspath(__file__), "--only", "traffic"]
            log(f"[bench] traffic pass: rocprofv3 --pmc {counter}")
            subprocess.run(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                           timeout=150, check=False)
            means[counter] = _counter_means(outdir, counter)
            shutil.rmtree(outdir, ignore_errors=True)
    except Exception as e:             # the bench line must not depend on the profiler
        return {"traffic": None, "traffic_note": f"counter pass failed: {e}"}
    f_scale = COPY_BYTES / (means["FETCH_SIZE"]["copy"] * 1024)
    w_scale = COPY_BYTES / (means["WRITE_SIZE"]["copy"] * 1024)
    traffic = 1024 * (means["FETCH_SIZE"]["attn"] * f_scale + means["WRITE_SIZE"]["attn"] * w_scale)
    return {"traffic": int(round(traffic)),
            "traffic_note": (f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE in this run: "
                             f"{means['FETCH_SIZE']['attn']:.1f} / {means['WRITE_SIZE']['attn']:.1f} "
                             f"KiB per dispatch, scaled x{f_scale:.3f} / x{w_scale:.3f} (512 MiB copy); "
                             f"{traffic / algo_bytes:.4f} x algorithmic bytes")}


# --------------------------------------------------------------------------
# CPU baselines (the reference's CPU path, restated; test infrastructure)
# --------------------------------------------------------------------------
def host_info():
    """The host the CPU baselines ran on: CPU model, logical CPUs, the CPUs
    this process may use, and torch's intra-op threads."""
    import torch
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"cpu_model": model, "nproc": os.cpu_count(), "usable_cpus": usable,
            "torch_threads": torch.get_num_threads()}


def _timed(fn, budget_s, max_n):
    """Seconds per call of fn(), over about budget_s of calls after one
    untimed call."""
    fn()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s and n < max_n:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def cpu_attention_baseline(k, v, Hq, Tq, G, Gv, B_total, budget_s=8.0):
    """What the reference does per decode step on the CPU: HF-style fp32
    attention (repeat_kv, QK^T*scale, softmax, PV) over the dequantised
    history + fp32 residual served by get_full_cache()
    (src/kivi_sycl/cache/manager.py:251-290).  ``k``/``v [nb, Hkv, T, D]``
    are the first nb sequences of the GPU workload (the same bits); the
    first Tq tokens are served through the oracle round-trip.  Timed with
    all host threads, reported in the same algorithmic-bytes unit."""
    import torch
    from oracle import codec
    nb, Hkv, T, D = k.shape
    Tr = T - Tq
    kh = k[:, :, :Tq].reshape(nb, Hkv, Tq // G, G, D).transpose(3, 4).contiguous()
    kh = torch.from_numpy(codec.roundtrip_groups(kh.numpy(), G).reshape(kh.shape))
    kh = kh.transpose(3, 4).reshape(nb, Hkv, Tq, D)
    vh = torch.from_numpy(codec.roundtrip_groups(v[:, :, :Tq].contiguous().numpy(), Gv)
                          .reshape(nb, Hkv, Tq, D))
    K = torch.cat([kh, k[:, :, Tq:]], dim=2)
    V = torch.cat([vh, v[:, :, Tq:]], dim=2)
    q = torch.randn(nb, Hq, 1, D, generator=torch.Generator().manual_seed(7)) * D ** -0.5
    rep = Hq // Hkv

    def step():
        Kx = K[:, :, None].expand(nb, Hkv, rep, T, D).reshape(nb, Hq, T, D)
        Vx = V[:, :, None].expand(nb, Hkv, rep, T, D).reshape(nb, Hq, T, D)
        w = torch.matmul(q, Kx.transpose(-1, -2)) * D ** -0.5
        w = torch.softmax(w, dim=-1)
        return torch.matmul(w, Vx)

    nbytes = attn_bytes(nb, Hq, Hkv, D, Tq, Tr, G, Gv)
    threads = torch.get_num_threads()
    dt, n = _timed(step, budget_s, 10000)
    torch.set_num_threads(1)
    try:
        dt1, n1 = _timed(step, budget_s / 2, 10000)
    finally:
        torch.set_num_threads(threads)
    return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": threads,
            "kind": "port", "single_thread": round(nbytes / dt1 / 1e9, 4),
            "host": host_info(),
            "sample": f"{nb} of {B_total} sequences x {Hkv} kv heads of the same K/V, context "
                      f"{T} (Tq={Tq}, Tr={Tr}): {n} steps in {n * dt:.1f}s on {threads} "
                      f"threads, {n1} steps in {n1 * dt1:.1f}s on 1 thread; torch fp32 "
                      f"attention over the dequantised history as the reference's HF model "
                      f"computes it on the CPU"}


def cpu_quantize_baseline(kt, v, G, B_total, budget_s=6.0):
    """The C oracle (one group per iteration, OpenMP over groups, the
    reference kernels' loop structure) on the first sequences of config 2's
    own K/V (``kt [nb,H,D,Seq]``, ``v [nb,H,Seq,D]``)."""
    from oracle import codec
    kn = kt.contiguous().numpy()
    vn = v.contiguous().numpy()
    nb, _, _, S = kt.shape

    def both():
        codec.quantize_groups(kn, G)
        codec.quantize_groups(vn, G)
    threads = codec.num_threads()
    dt, n = _timed(both, budget_s, 1000)
    codec.set_num_threads(1)
    try:
        dt1, n1 = _timed(both, budget_s / 2, 1000)
    finally:
        codec.set_num_threads(threads)
    return {"value": nb * S / dt / 1e6, "unit": "Mtokens/s", "cores": threads,
            "kind": "port", "single_thread": round(nb * S / dt1 / 1e6, 4),
            "host": host_info(),
            "sample": f"keys {list(kt.shape)} + values {list(v.shape)} ({nb} of {B_total} "
                      f"sequences of config 2's K/V): {n} passes in {n * dt:.1f}s on "
                      f"{threads} threads, {n1} in {n1 * dt1:.1f}s on 1 thread"}


def cache_loop(cache, k_all, v_all, layers, sync=None):
    """Config 1's cache workload: one new token per layer per decode step,
    fed to ``cache`` as a transformers model feeds it in generate()
    (src/kivi_sycl/generation/generate.py:70-82): the served view
    (get_full_cache), the model's in-place update of every layer, then
    add_tokens.  Returns seconds per step."""
    from transformers import DynamicCache
    T = k_all.shape[2]
    if sync:
        sync()
    t0 = time.perf_counter()
    for t in range(T):
        view = cache.get_full_cache() if t else DynamicCache()
        for layer in range(layers):
            view.update(k_all[:, :, t:t + 1], v_all[:, :, t:t + 1], layer)
        cache.add_tokens(view)
    if sync:
        sync()
    return (time.perf_counter() - t0) / T


def cpu_cache_baseline(layers, B, H, D, G, R, T, reps=3):
    """The reference's KiviCache CPU path restated (oracle/kivi_cache.py,
    src/kivi_sycl/cache/manager.py:162-374, with the C oracle codec as its
    round-trip) over config 1's workload; best of ``reps`` runs."""
    import torch
    from oracle.kivi_cache import KiviCacheOracle
    k, v = synth_kv(B, H, T, D, 1234 + 1)
    best = min(cache_loop(KiviCacheOracle(layers, D, None, G, R), k, v, layers)
               for _ in range(reps))
    return {"value": round(1.0 / best, 2), "unit": "decode steps/s",
            "us_per_step": round(best * 1e6, 1), "cores": torch.get_num_threads(),
            "kind": "port", "host": host_info(),
            "sample": f"config 1: {layers} layers, B={B}, H={H}, D={D}, G={G}, R={R}, {T} "
                      f"decode steps of one token from empty (best of {reps}); the CPU "
                      f"KiviCache with its fp32 history and the codec round-trip per flush"}


# --------------------------------------------------------------------------
# End to end: the reference's one published figure (README.md:12-20, method
# examples/benchmark.py:21-145): GPT-2 greedy decoding of 200 tokens with an
# unquantised DynamicCache against the KIVI cache (G=32, R=64).
# --------------------------------------------------------------------------
GPT2_EOS = 50256


def e2e_gpt2(dev, n_tokens=200, G=32, R=64, prompt_len=40, reps=3, log=print):
    """Seeded random-init GPT-2-small (12 layers, 12 heads, head_dim 64) in
    fp32 on the GPU (no checkpoint exists offline), a seeded prompt of
    ``prompt_len`` token ids (no tokenizer: the reference's default prompt is
    about that long), three arms timed as benchmark.py times them:
    * fp32: model() with HF's DynamicCache, ``n_tokens`` calls from the
      prompt, greedy, the end-of-text check every step (benchmark.py:44-57);
    * kivi: this package's KiviCache (codes, scales, zeros and the residual
      window in HBM) driven as the reference's generate() drives its cache,
      the prefill untimed and ``n_tokens - 1`` steps timed
      (benchmark.py:70-104);
    * kivi_packed: generate_packed()'s loop, attention read straight from
      the 2-bit store by the fused kernel, timed the same way.
    Each arm runs once untimed first, at full length (kernels first launched
    at a flush load on their first call), then ``reps`` timed runs with the
    arms in turn; the median run is reported.  tok/s = tokens produced /
    timed seconds (benchmark.py:99-134)."""
    import torch
    from transformers import GPT2Config, GPT2LMHeadModel
    from intel_kivi_hybrid_amd import KiviCache, KiviPackedCache
    from intel_kivi_hybrid_amd.cache.packed_cache import packed_attention
    torch.manual_seed(0)
    model = GPT2LMHeadModel(GPT2Config(n_layer=12, n_head=12, n_embd=768)).eval().to(dev)
    ids = torch.randint(0, model.config.vocab_size, (1, prompt_len),
                        generator=torch.Generator().manual_seed(1)).to(dev)
    nxt = lambda out: out.logits[:, -1, :].argmax(dim=-1).unsqueeze(1)   # noqa: E731

    @torch.no_grad()
    def fp32(n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        inp, past, toks = ids, None, []
        for _ in range(n):
            out = model(inp, past_key_values=past, use_cache=True)
            past = out.past_key_values
            inp = nxt(out)
            toks.append(inp)
            if inp.item() == GPT2_EOS:
                break
        torch.cuda.synchronize()
        return toks, time.perf_counter() - t0, None

    @torch.no_grad()
    def kivi(n):
        cache = KiviCache.from_model(model, device=dev, group_size=G, residual_length=R)
        out = model(ids, use_cache=True)
        cache.add_tokens(out.past_key_values)
        inp = nxt(out)
        toks = [inp]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(1, n):
            out = model(inp, past_key_values=cache.get_full_cache(), use_cache=True)
            cache.add_tokens(out.past_key_values)
            inp = nxt(out)
            toks.append(inp)
            if inp.item() == GPT2_EOS:
                break
        torch.cuda.synchronize()
        return toks, time.perf_counter() - t0, cache

    @torch.no_grad()
    def kivi_packed(n):
        cache = KiviPackedCache.from_model(model, device=dev, group_size=G, residual_length=R)
        with packed_attention(model):
            out = model(ids, past_key_values=cache, use_cache=True)
            inp = nxt(out)
            toks = [inp]
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(1, n):
                out = model(inp, past_key_values=cache, use_cache=True)
                inp = nxt(out)
                toks.append(inp)
                if inp.item() == GPT2_EOS:
                    break
            torch.cuda.synchronize()
        return toks, time.perf_counter() - t0, cache

    arms = (("fp32", fp32), ("kivi", kivi), ("kivi_packed", kivi_packed))
    for _, arm in arms:
        arm(n_tokens)       # untimed, whole length: kernels first launched at a flush load here
    times, runs = {name: [] for name, _ in arms}, {}
    for _ in range(reps):   # the arms in turn, so that clock drift spreads over all three
        for name, arm in arms:
            toks, dt, cache = arm(n_tokens)
            times[name].append(dt)
            runs[name] = (toks, cache)
    res, ref_ids = {}, None
    for name, _ in arms:
        toks, cache = runs[name]
        dt = sorted(times[name])[len(times[name]) // 2]
        tids = torch.cat(toks, dim=1)[0].cpu()
        r = {"tokens": len(toks), "seconds": round(dt, 4), "tok_s": round(len(toks) / dt, 2),
             "ms_per_token": round(dt / len(toks) * 1e3, 3),
             "seconds_all": [round(t, 4) for t in times[name]]}
        if ref_ids is None:
            ref_ids = tids
        else:
            m = min(len(ref_ids), len(tids))
            same = (ref_ids[:m] == tids[:m])
            r["token_match_vs_fp32"] = round(same.float().mean().item(), 4)
            r["first_divergence"] = int(m if bool(same.all()) else (~same).nonzero()[0, 0])
            # benchmark.py:124-131: speedup or overhead against the fp32 arm
            ratio = res["fp32"]["tok_s"] / r["tok_s"]
            r["overhead_pct_vs_fp32"] = round((ratio - 1) * 100, 1)
            s0 = cache.get_stats(0)
            r["layer0_kivi_bytes"], r["layer0_fp32_bytes"] = s0["kivi_bytes"], s0["fp32_bytes"]
            r["compression"] = round(s0["compression"], 3)
        res[name] = r
        log(f"[bench] e2e gpt2 {name}: {r}")
    res["config"] = {"model": "GPT-2-small shape (12 layers, 12 heads, head_dim 64), seeded "
                              "random init, fp32, on the GPU", "prompt_tokens": prompt_len,
                     "new_tokens": n_tokens, "group_size": G, "residual": R,
                     "timed_runs": reps}
    return res


# --------------------------------------------------------------------------
# End to end at serving scale: config 4's attention geometry inside a
# Llama-3-8B-shaped model (no reference figure: the reference times GPT-2 only).
# --------------------------------------------------------------------------
def e2e_llama(dev, B=16, context=8192, steps=32, layers=4, G=32, R=128, reps=3, log=print):
    """Seeded random-init Llama-3-8B shape (hidden 4096, MLP 14336, 32 query /
    8 kv heads, head_dim 128, vocab 128256) cut to ``layers`` layers, bf16 on
    the GPU; B sequences of ``context`` seeded prompt tokens, then ``steps``
    decode steps of one token per sequence, the same seeded tokens in every
    arm (identical work per arm and comparable final logits: a random-init
    model's greedy choices part at the first small difference), timed for
    four caches:
    * bf16 ``DynamicCache`` (transformers' default: K/V concatenated every
      step, SDPA over them);
    * bf16 ``StaticCache`` (preallocated for context + steps, SDPA over the
      whole buffer with a mask);
    * ``KiviPackedCache`` (2-bit store, bf16 residual ring of R tokens, the
      packed attention kernel; the prompt attends with SDPA, as in the other
      arms, and is then quantised);
    * ``KiviCache`` driven as the reference's generate() drives it
      (get_full_cache() before each forward, add_tokens() after): the same
      KIVI arithmetic served as a dequantised bf16 cache to SDPA, so the
      packed arm's logits are also compared with it.
    Each arm: the prompt forward untimed (last position's logits only), then
    ``steps`` forwards of one token per sequence with no host sync inside the
    timed region; one untimed run, then ``reps`` timed runs with the arms in
    turn, the median reported.  tok/s = B * steps / seconds.  Fidelity
    against the bf16 ``DynamicCache``: max |logit difference| / max |logit|
    and the mean cosine similarity of the final step's logits rows, and the
    same of the packed arm against the served KIVI cache (the same
    quantisation).  On a random-init model 2-bit K/V move the logits far
    more than on a trained one: its attention spreads over hundreds of
    tokens of zero-mean values, so the output is of the order of the
    quantisation noise averaged over them; both KIVI arms differ from bf16
    alike and agree with each other."""
    import torch
    from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM, StaticCache
    from intel_kivi_hybrid_amd import KiviCache, KiviPackedCache
    from intel_kivi_hybrid_amd.cache.packed_cache import packed_attention
    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336,
                      num_hidden_layers=layers, num_attention_heads=32, num_key_value_heads=8,
                      max_position_embeddings=context + steps + 8, rope_theta=500000.0)
    model = LlamaForCausalLM(cfg).eval().to(dev, torch.bfloat16)
    ids = torch.randint(0, cfg.vocab_size, (B, context),
                        generator=torch.Generator().manual_seed(1)).to(dev)
    dec = torch.randint(0, cfg.vocab_size, (B, steps),
                        generator=torch.Generator().manual_seed(2)).to(dev)

    def static_cache():
        return StaticCache(config=cfg, max_cache_len=context + steps)

    def packed_cache():
        return KiviPackedCache.from_model(model, device=dev, group_size=G, residual_length=R)

    @torch.no_grad()
    def run_served():
        cache = KiviCache.from_model(model, device=dev, group_size=G, residual_length=R)
        pos = torch.arange(context + steps, device=dev)
        out = model(ids, use_cache=True, cache_position=pos[:context], logits_to_keep=1)
        cache.add_tokens(out.past_key_values)
        del out
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            out = model(dec[:, i:i + 1], past_key_values=cache.get_full_cache(), use_cache=True,
                        cache_position=pos[context + i:context + i + 1])
            cache.add_tokens(out.past_key_values)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        return out.logits[:, -1].float(), dt, cache

    @torch.no_grad()
    def run(make, packed):
        if make is None:
            return run_served()
        ctx = packed_attention(model) if packed else contextlib.nullcontext()
        with ctx:
            cache = make()
            pos = torch.arange(context + steps, device=dev)      # positions made up front
            model(ids, past_key_values=cache, use_cache=True, cache_position=pos[:context],
                  logits_to_keep=1)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(steps):
                out = model(dec[:, i:i + 1], past_key_values=cache, use_cache=True,
                            cache_position=pos[context + i:context + i + 1])
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
        return out.logits[:, -1].float(), dt, cache

    arms = (("bf16_dynamic", DynamicCache, False), ("bf16_static", static_cache, False),
            ("kivi_packed", packed_cache, True), ("kivi_served", None, False))
    for _, make, packed in arms:
        run(make, packed)
        torch.cuda.empty_cache()
    times, logits_of, caches = {n: [] for n, _, _ in arms}, {}, {}
    for _ in range(reps):
        for name, make, packed in arms:
            logits, dt, cache = run(make, packed)
            times[name].append(dt)
            logits_of[name] = logits
            if name.startswith("kivi"):
                caches[name] = cache.get_stats(0)
            del cache
            torch.cuda.empty_cache()
    kv_bf16 = 2 * B * cfg.num_key_value_heads * (context + steps) * 128 * 2
    res = {}
    for name, _, _ in arms:
        dt = sorted(times[name])[len(times[name]) // 2]
        r = {"ms_per_step": round(dt / steps * 1e3, 3), "tok_s": round(B * steps / dt, 1),
             "seconds_all": [round(t, 4) for t in times[name]]}
        if name != "bf16_dynamic":
            ref, got = logits_of["bf16_dynamic"], logits_of[name]
            err = ((got - ref).abs().max() / ref.abs().max()).item()
            r["logits_rel_err_vs_dynamic"] = float(f"{err:.3e}")
            r["logits_cosine_vs_dynamic"] = round(
                torch.nn.functional.cosine_similarity(got, ref, dim=-1).mean().item(), 6)
            r["speedup_vs_dynamic"] = round(sorted(times["bf16_dynamic"])[reps // 2] / dt, 3)
        if name == "kivi_packed":
            ref, got = logits_of["kivi_served"], logits_of[name]
            err = ((got - ref).abs().max() / ref.abs().max()).item()
            r["logits_rel_err_vs_served"] = float(f"{err:.3e}")
            r["logits_cosine_vs_served"] = round(
                torch.nn.functional.cosine_similarity(got, ref, dim=-1).mean().item(), 6)
        if name in caches:          # the KIVI accounting of get_stats (2-bit store + window)
            r["layer0_kivi_bytes"] = caches[name]["kivi_bytes"]
        else:
            r["layer0_kv_bytes"] = kv_bf16
        res[name] = r
        log(f"[bench] e2e llama {name}: {r}")
    res["config"] = {"model": f"Llama-3-8B shape cut to {layers} layers (hidden 4096, MLP 14336, "
                              f"32/8 heads, head_dim 128, vocab 128256), seeded random init, "
                              f"bf16, on the GPU", "batch": B, "prompt_tokens": context,
                     "decode_steps": steps, "group_size": G, "residual": R, "timed_runs": reps}
    del model
    return res


# --------------------------------------------------------------------------
CONFIG4 = (64, 32, 8, 128, 8192, 128, 32)      # B, Hq, Hkv, D, context, R, G
PRECISION = ("fp32 inputs and outputs; 2-bit codes with fp32 scales/zeros, bit-exact to the "
             "reference codec; attention products on bf16 matrix cores with fp32 accumulation, "
             "the codes exact as subnormal bf16 operands, each fp32 key factor split into three "
             "bf16 pieces (~2^-25 relative; two, ~2^-17, at 8 query heads per kv head) and each "
             "value factor into two (~2^-17); softmax and residual window in fp32")
DTYPE = "fp32 I/O; bf16 split-factor MFMA products; fp32 accumulation"


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--attn-iters", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter passes behind roofline.traffic")
    ap.add_argument("--only", choices=["config4", "attention", "gqa8", "ring16", "b1",
                                       "config3", "config5", "codec", "prefill", "copy",
                                       "traffic", "cache1", "e2e", "e2e_llama"],
                    default=None,
                    help="run one workload (for profiling); 'gqa8' is attention of 64 query "
                         "heads over config 4's store (8 query heads per kv head); 'ring16' "
                         "is config-4 attention over a store whose residual ring is bf16 (a "
                         "bf16 model's packed cache); 'b1' is config 4's shape for one "
                         "sequence (B=1: the split plan and its merge) and for 16 and 24 "
                         "sequences; 'copy' is "
                         "a plain 512 MiB device copy for calibrating the FETCH_SIZE / "
                         "WRITE_SIZE counters; 'traffic' is the workload of the counter passes; "
                         "'cache1' is config 1's KiviCache loop; 'e2e' is GPT-2 greedy "
                         "decoding with and without the KIVI cache; 'e2e_llama' is greedy "
                         "decoding of a 4-layer Llama-3-8B-shaped bf16 model at B=16, 8K "
                         "context with transformers' caches and the packed cache")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the KIVI hot path here is built and "
              "measured on a single MI355X (no multi-GPU path); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    log = lambda *a: print(*a, file=sys.stderr, flush=True)      # noqa: E731
    only = args.only
    W, K = args.warmup, args.steps

    if only == "copy":
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(7)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy: {COPY_BYTES} bytes read and written per launch, 5 launches")
        return
    if only == "traffic":
        traffic_workload(dev)
        return

    extra = {}
    loop = attn4 = None
    # ---- config 4: the headline decode loop -------------------------------
    if only in (None, "config4", "attention", "gqa8", "ring16"):
        B, Hq, Hkv, D, T, R, G = CONFIG4
        Tq = T - R
        # the store starts Tr0 tokens into its window so that the first timed
        # step fills it to R and flushes
        Tr0 = (R - 1) - (W % G)
        n_new = W + K
        log(f"[bench] config4: B={B} Hq={Hq} Hkv={Hkv} D={D} context {T} R={R} G={G}; "
            f"making K/V on the CPU")
        k, v = synth_kv(B, Hkv, store_tokens(Tq, Tr0, G, R) + n_new, D, 1234 + 4)
        st = make_store(k[:, :, :Tq + Tr0], v[:, :, :Tq + Tr0], G, G, R, dev,
                        extra_chunks=n_new // G + 2)
        k_new = k[:, :, Tq + Tr0:].to(dev)
        v_new = v[:, :, Tq + Tr0:].to(dev)
        cpu_k4 = k[:4, :, :T].clone()
        cpu_v4 = v[:4, :, :T].clone()
        st16 = q16 = None
        if only in (None, "ring16"):
            # the same context with a bf16 residual ring, as a bf16 model's
            # KiviPackedCache keeps it: bf16 K/V quantised, window in bf16
            # (built now, from the CPU K/V; timed after the headline calls)
            from intel_kivi_hybrid_amd.store import PackedKVStore
            st16 = PackedKVStore(B, Hkv, D, G, R, dev, group_size_v=G,
                                 chunk_capacity=T // G + 4, residual_dtype=torch.bfloat16)
            k16, v16 = k[:, :, :T].to(dev, torch.bfloat16), v[:, :, :T].to(dev, torch.bfloat16)
            st16.extend(k16[:, :, :T - 1], v16[:, :, :T - 1], flush_at=R)
            st16.append(k16[:, :, T - 1:], v16[:, :, T - 1:])
            del k16, v16
            assert (st16.quantized_tokens, st16.res_len) == (Tq, R)
            q16 = (torch.randn(B, Hq, D, generator=torch.Generator().manual_seed(16))
                   * D ** -0.5).to(dev)
        del k, v
        gq = torch.Generator().manual_seed(5)
        q_all = (torch.randn(n_new, B, Hq, D, generator=gq) * D ** -0.5).to(dev)
        q4 = (torch.randn(B, Hq, D, generator=gq) * D ** -0.5).to(dev)
        # roofline: the attention kernel alone at context T (Tq = T - R
        # quantised, a full window of R), the first tokens of the loop filling it
        m = R - Tr0
        st.append(k_new[:, :, :m], v_new[:, :, :m])
        if only not in ("gqa8", "ring16"):
            attn4 = time_attention(st, q4, args.attn_iters)
            log(f"[bench] config4 attention: {attn4['avg_us']:.1f} us, {attn4['gbs']:.0f} GB/s "
                f"(Tq={attn4['Tq']}, Tr={attn4['Tr']}, splits={attn4['splits']})")
        if only in (None, "gqa8"):
            # the same store read by 64 query heads: 8 per kv head, the
            # Llama-3-70B grouping (not a benchmark config)
            q8 = (torch.randn(B, 8 * Hkv, D, generator=torch.Generator().manual_seed(8))
                  * D ** -0.5).to(dev)
            a8 = time_attention(st, q8, args.attn_iters)
            log(f"[bench] gqa8 attention (B={B}, {8 * Hkv}/{Hkv} heads, config 4's store): "
                f"{a8['avg_us']:.1f} us, {a8['gbs']:.0f} GB/s (splits={a8['splits']})")
            extra["attention_gqa8"] = {k_: a8[k_] for k_ in ("avg_us", "gbs", "Tq", "Tr",
                                                             "splits")}
            del q8
        if st16 is not None:
            a16 = time_attention(st16, q16, args.attn_iters)
            log(f"[bench] config4 attention, bf16 residual ring: {a16['avg_us']:.1f} us, "
                f"{a16['gbs']:.0f} GB/s (Tq={a16['Tq']}, Tr={a16['Tr']})")
            extra["attention_config4_ring_bf16"] = {k_: a16[k_] for k_ in ("avg_us", "gbs", "Tq",
                                                                           "Tr")}
            del st16, q16
            torch.cuda.empty_cache()
        st.rollback(m)
        if only in ("attention", "gqa8", "ring16"):
            return
        flush4 = time_flush(st)
        log(f"[bench] config4 flush: {flush4['avg_us']:.1f} us, {flush4['gbs']:.0f} GB/s")
        loop = decode_loop(st, q_all, k_new, v_new, K, W, R)
        log(f"[bench] config4 decode loop: {loop['ms_per_step'] * 1e3:.1f} us/step, "
            f"{loop['gbs']:.0f} GB/s, {loop['flushes']} flushes in {K} steps, context "
            f"{loop['context'][0]}..{loop['context'][1]} (host issues a step in "
            f"{loop['submit_s'] / K * 1e6:.1f} us)")
        extra["flush_config4"] = {k_: round(flush4[k_], 2) for k_ in ("avg_us", "gbs")}
        del st, k_new, v_new, q_all
        torch.cuda.empty_cache()
        if only == "config4":
            return

    if only in (None, "b1"):
        # ---- one sequence at config 4's shape: 8 (b, kv-head) pairs, so the
        # plan splits the context (32 splits) and merges the partials
        B1, Hq1, H1, D1, T1, R1, G1 = 1, *CONFIG4[1:]
        k, v = synth_kv(B1, H1, T1, D1, 1234 + 41)
        s1 = make_store(k[:, :, :T1 - 1], v[:, :, :T1 - 1], G1, G1, R1, dev)
        s1.append(k[:, :, -1:].to(dev), v[:, :, -1:].to(dev))
        del k, v
        q = (torch.randn(B1, Hq1, D1, generator=torch.Generator().manual_seed(41))
             * D1 ** -0.5).to(dev)
        a1 = time_attention(s1, q, args.attn_iters)
        log(f"[bench] one sequence (B=1, config 4's heads, context {T1}): {a1['avg_us']:.1f} us "
            f"per call, {a1['splits']} splits + merge")
        extra["attention_b1"] = {k_: a1[k_] for k_ in ("avg_us", "gbs", "Tq", "Tr", "splits")}
        del s1
        # the first steps of a sequence: a 100-token context, all of it still
        # in the residual window (no chunk yet)
        k, v = synth_kv(B1, H1, 100, D1, 1234 + 42)
        s0 = make_store(k, v, G1, G1, R1, dev)
        assert (s0.n_chunks, s0.res_len) == (0, 100)
        a0 = time_attention(s0, q, args.attn_iters)
        log(f"[bench] one sequence, 100 tokens all in the window: {a0['avg_us']:.1f} us per call")
        extra["attention_b1_window_only"] = {k_: a0[k_] for k_ in ("avg_us", "Tq", "Tr")}
        del s0, k, v
        # mid batches at config 4's heads and context (the split plan's
        # middle ground: 4 and 2 splits), each with a second store called
        # in turn so that the MALL cannot serve the bytes
        for Bm in (16, 24):
            k, v = synth_kv(Bm, H1, T1, D1, 1234 + 43 + Bm)
            sts = []
            for _ in range(3 if Bm == 16 else 2):
                s_ = make_store(k[:, :, :T1 - 1], v[:, :, :T1 - 1], G1, G1, R1, dev)
                s_.append(k[:, :, -1:].to(dev), v[:, :, -1:].to(dev))
                sts.append(s_)
            del k, v
            qm = (torch.randn(Bm, Hq1, D1, generator=torch.Generator().manual_seed(43))
                  * D1 ** -0.5).to(dev)
            am = time_attention(sts[0], qm, args.attn_iters, rotate=sts[1:])
            log(f"[bench] B={Bm} (config 4's heads, context {T1}): {am['avg_us']:.1f} us per "
                f"call, {am['gbs']:.0f} GB/s, {am['splits']} splits")
            extra[f"attention_b{Bm}"] = {k_: am[k_] for k_ in ("avg_us", "gbs", "Tq", "Tr",
                                                              "splits")}
            del sts
        torch.cuda.empty_cache()

    if only in (None, "config3"):
        # ---- config 3: MHA, 4096 quantised + 128 residual tokens -----------
        B3, H3, D3, R3, G3 = 16, 32, 128, 128, 32
        k, v = synth_kv(B3, H3, 4096 + R3, D3, 1234 + 3)
        # two copies of the 336 MB store, called in turn (> 512 MB between
        # two reads of one copy, so the MALL cannot serve them)
        sts = []
        for _ in range(2):
            s3 = make_store(k[:, :, :4096 + R3 - 1], v[:, :, :4096 + R3 - 1], G3, G3, R3, dev)
            s3.append(k[:, :, -1:].to(dev), v[:, :, -1:].to(dev))
            sts.append(s3)
        del k, v
        q = (torch.randn(B3, H3, D3, generator=torch.Generator().manual_seed(6))
             * D3 ** -0.5).to(dev)
        a3 = time_attention(sts[0], q, args.attn_iters, rotate=sts[1:])
        log(f"[bench] config3 attention: {a3['avg_us']:.1f} us, {a3['gbs']:.0f} GB/s "
            f"(Tq={a3['Tq']}, Tr={a3['Tr']}; two stores in turn)")
        extra["attention_config3"] = {k_: a3[k_] for k_ in ("avg_us", "gbs", "Tq", "Tr", "splits")}
        del sts
        torch.cuda.empty_cache()

    if only in (None, "config5"):
        # ---- config 5: 131072 quantised tokens, Gv=128, split-K + merge ----
        B5, Hq5, H5, D5, R5, G5, Gv5 = 4, 32, 8, 128, 128, 32, 128
        k, v = synth_kv(B5, H5, 131072 + R5, D5, 1234 + 5)
        # two copies of the 441 MB store, called in turn (see config 3)
        sts = []
        for _ in range(2):
            s5 = make_store(k[:, :, :131072 + R5 - 1], v[:, :, :131072 + R5 - 1], G5, Gv5, R5,
                            dev)
            s5.append(k[:, :, -1:].to(dev), v[:, :, -1:].to(dev))
            sts.append(s5)
        st = sts[0]
        del k, v
        q = (torch.randn(B5, Hq5, D5, generator=torch.Generator().manual_seed(7))
             * D5 ** -0.5).to(dev)
        a5 = time_attention(st, q, args.attn_iters, rotate=sts[1:])
        f5 = time_flush(st)
        step_us = a5["avg_us"] + f5["avg_us"]
        log(f"[bench] config5 attention: {a5['avg_us']:.1f} us, {a5['gbs']:.0f} GB/s "
            f"(Tq={a5['Tq']}, Tr={a5['Tr']}, {a5['splits']} splits + merge); flush "
            f"{f5['avg_us']:.1f} us; decode step {step_us:.1f} us")
        extra["attention_config5"] = {k_: a5[k_] for k_ in ("avg_us", "gbs", "Tq", "Tr", "splits")}
        extra["attention_config5"].update({
            "flush_us": round(f5["avg_us"], 2), "step_us": round(step_us, 2),
            "step_gbs": round((a5["bytes"] + f5["bytes"]) / (step_us * 1e-6) / 1e9, 1)})
        del st, sts
        torch.cuda.empty_cache()

    if only in (None, "cache1"):
        # ---- config 1: the KiviCache loop (12 layers, B=1, H=12, D=64,
        # R=G=32, 200 steps of one token from empty), cache in HBM
        from intel_kivi_hybrid_amd import KiviCache
        L1, B1, H1, D1, G1, R1, T1 = 12, 1, 12, 64, 32, 32, 200
        k, v = synth_kv(B1, H1, T1, D1, 1234 + 1)
        k, v = k.to(dev), v.to(dev)
        runs = []
        for _ in range(3):
            c1 = KiviCache(L1, D1, None, device=dev, group_size=G1, residual_length=R1)
            runs.append(cache_loop(c1, k, v, L1, sync=torch.cuda.synchronize))
        s1 = c1.get_stats(0)
        extra["cache_config1"] = {
            "us_per_step": round(min(runs) * 1e6, 1), "steps_per_s": round(1 / min(runs), 1),
            "layers": L1, "steps": T1, "flushes": c1.total_flushes,
            "layer0_kivi_bytes": s1["kivi_bytes"], "layer0_fp32_bytes": s1["fp32_bytes"],
            "compression": round(s1["compression"], 3),
            "note": "best of 3 runs; each step: get_full_cache, the model's in-place update "
                    "of 12 layers (HF DynamicCache), add_tokens with its flushes"}
        log(f"[bench] config1 KiviCache loop (HBM): {extra['cache_config1']}")
        del k, v, c1
        if only == "cache1":
            if not args.no_cpu_baseline:
                log(f"[bench] cpu baseline cache: {cpu_cache_baseline(L1, B1, H1, D1, G1, R1, T1)}")
            return

    if only in (None, "e2e"):
        extra["e2e_gpt2"] = e2e_gpt2(dev, log=log)
        torch.cuda.empty_cache()
        if only == "e2e":
            return

    if only in (None, "e2e_llama"):
        extra["e2e_llama"] = e2e_llama(dev, log=log)
        torch.cuda.empty_cache()
        if only == "e2e_llama":
            return

    qb = None
    cpu_kt2 = cpu_v2 = None
    if only in (None, "codec", "prefill"):
        # ---- config 2: the _C codec ops and the batched prefill flush -------
        B2, H2, S2, D2, G2 = 8, 32, 4096, 128, 32
        k, v = synth_kv(B2, H2, S2, D2, 1234 + 2)
        if only in (None, "codec"):
            kt = k.transpose(2, 3).contiguous()
            cpu_kt2, cpu_v2 = kt[:1].clone(), v[:1].clone()
            qb = codec_bench(kt.to(dev), v.to(dev), G2)
            del kt
            for name in ("quantize", "dequantize", "roundtrip"):
                r = qb[name]
                log(f"[bench] config2 {name} K+V: {r['us_per_pair']:.1f} us, {r['gbs']:.0f} GB/s, "
                    f"{r['mtokens_s']:.1f} Mtokens/s")
            torch.cuda.empty_cache()
        if only in (None, "prefill"):
            pf = prefill_bench(k, v, dev)
            for name, r in pf.items():
                log(f"[bench] prefill flush ({name} K/V, {S2}-token prompt, B={B2}, {H2} heads): "
                    f"{r['us']:.1f} us, {r['gbs']:.0f} GB/s, {r['mtokens_s']:.1f} Mtokens/s")
            extra["prefill_flush"] = pf
        del k, v
        torch.cuda.empty_cache()
    if only is not None:
        return

    B, Hq, Hkv, D, T, R, G = CONFIG4
    cpu = cpu_q = cpu_c = None
    if not args.no_cpu_baseline:
        cpu = cpu_attention_baseline(cpu_k4, cpu_v4, Hq, T - R, G, G, B)
        log(f"[bench] cpu baseline attention: {cpu}")
        cpu_q = cpu_quantize_baseline(cpu_kt2, cpu_v2, 32, 8)
        log(f"[bench] cpu baseline quantize: {cpu_q}")
        cpu_c = cpu_cache_baseline(12, 1, 12, 64, 32, 32, 200)
        log(f"[bench] cpu baseline cache: {cpu_c}")
    traffic = {"traffic": None, "traffic_note": "not measured (--no-traffic)"}
    if not args.no_traffic:
        traffic = measure_traffic(attn4["bytes"], log)
        log(f"[bench] traffic: {traffic}")

    line = {
        "metric": "packed-KV decode attention GB/s (% HBM peak) + quantize Mtokens/s, 1 GPU",
        "value": round(loop["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(loop["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE,
        "precision": PRECISION,
        "data": "synthetic: seeded N(0,1) K/V made on the CPU (4 key channels x10 per kv "
                "head, 2% of value tokens x8 per sequence and head), copied to HBM before "
                "timing; the CPU baselines use the same bits",
        "config": {"workload": "config4 Llama-3-8B GQA packed-KV decode loop",
                   "batch": B, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D,
                   "context": T, "residual": R, "group_size": G,
                   "step": "attention with the new token appended in the same launch + flush "
                           "of the 32 oldest residual tokens when the window reaches R",
                   "flushes": loop["flushes"],
                   "context_range": loop["context"]},
        "pct_hbm_peak": round(100 * loop["gbs"] / HBM_PEAK_GBS, 2),
        "quantize_mtokens_s": qb["quantize"]["mtokens_s"],
        "quantize_gbs": qb["quantize"]["gbs"],
        "quantize_config": "config2 keys [8,32,128,4096] G=32 + values [8,32,4096,128] G=32",
        "codec_config2": {k_: qb[k_] for k_ in ("quantize", "dequantize", "roundtrip")},
        "quantize_max_err_over_scale": round(qb["max_err_over_scale"], 4),
        "roofline": {"bound": "hbm", "achieved": round(attn4["gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(attn4["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic["traffic"], "traffic_note": traffic["traffic_note"],
                     "kernel": "attn_mfma_kernel<4,128,32,4,false>, config 4, one call "
                               f"(Tq={attn4['Tq']}, Tr={attn4['Tr']})",
                     "avg_us": round(attn4["avg_us"], 2), "bytes_per_launch": attn4["bytes"]},
        "cpu_baseline": cpu,
        "cpu_baseline_quantize": cpu_q,
        "cpu_baseline_cache": cpu_c,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
