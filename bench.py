"""KIVI hot-path benchmark on one MI355X.

Headline (``value``): packed-KV decode throughput at benchmark config 4
(Llama-3-8B GQA shape: B=64, 32 q heads / 8 kv heads, D=128, 8K context,
R=128, G=32).  One step = append the new token's K/V to the HBM residual
ring, flush 32 tokens into the packed store whenever the residual reaches R,
and run the fused packed decode attention for one query token per sequence.
``value`` is algorithmic bytes moved by those steps / wall time of the K timed
steps, in GB/s.

Also reported: the attention kernel alone against the 8 TB/s HBM roofline
(``roofline``), configs 3 and 5, the quantise microbench of config 2
(Mtokens/s), and CPU baselines of the reference path timed on the host.

Algorithmic bytes (per (batch, kv-head)):
  attention : D*Tq/4 + 8*D*Tq/Gk + Tq*D/4 + 8*Tq*D/Gv + 8*Tr*D + 8*(Hq/Hkv)*D
  flush     : 8*G*D (read residual) + G*D/4 + 8*D + G*D/4 + 8*G*D/Gv (write)
  append    : 8*D read + 8*D write
  quantise  : per tensor of N fp32: 4N read + N/4 + 8N/G written
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


# HBM bytes that one config-4 attention launch (Tq=8096, Tr=96; 583,008,256
# algorithmic bytes) moves: rocprofv3 --pmc FETCH_SIZE x 2.00 + WRITE_SIZE
# x 1.00 per dispatch, the factors calibrated on a 512 MiB copy
# (profiles/attn_mfma_config4.md).  Reported only for that exact workload.
ATTN4_ALGO_BYTES = 583_008_256
ATTN4_TRAFFIC_BYTES = 583_457_664


def attn_bytes(B, Hq, Hkv, D, Tq, Tr, Gk, Gv):
    per = (D * Tq // 4 + 8 * D * Tq // Gk + Tq * D // 4 + 8 * Tq * D // Gv
           + 8 * Tr * D + 8 * (Hq // Hkv) * D)
    return per * B * Hkv


def flush_bytes(B, Hkv, D, G, Gv):
    return B * Hkv * (8 * G * D + G * D // 4 + 8 * D + G * D // 4 + 8 * G * D // Gv)


def append_bytes(B, Hkv, D, n=1):
    return B * Hkv * 16 * D * n


def quant_bytes(N, G):
    return 4 * N + N // 4 + 8 * N // G


# --------------------------------------------------------------------------
# GPU workloads
# --------------------------------------------------------------------------
def synth_kv(B, H, T, D, seed, device):
    """N(0,1) K/V with 4 key channels x10 per head and 2% value tokens x8."""
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(B, H, T, D, generator=g, device=device)
    v = torch.randn(B, H, T, D, generator=g, device=device)
    ch = torch.randperm(D, generator=g, device=device)[:4]
    k[..., ch] *= 10.0
    tok = torch.randperm(T, generator=g, device=device)[:max(1, round(0.02 * T))]
    v[:, :, tok, :] *= 8.0
    return k, v


def build_store(B, Hkv, D, G, Gv, R, T, seed, device, extra_chunks=16):
    from intel_kivi_hybrid_amd.store import PackedKVStore
    st = PackedKVStore(B, Hkv, D, G, R, device, group_size_v=Gv,
                       chunk_capacity=T // G + extra_chunks)
    k, v = synth_kv(B, Hkv, T, D, seed, device)
    st.extend(k, v, flush_at=R)
    del k, v
    return st


def settle_clocks(fn, seconds=0.05, min_calls=20):
    """Runs fn back to back for ~`seconds` of GPU time (untimed).  From idle,
    MI355X clocks take tens of milliseconds to ramp up: timing without this
    reports the first calls ~20% slow."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while n < min_calls or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
        if n % 10 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_attention(st, Hq, iters, seed, device, blocks=5):
    """Average duration of one fused-attention call and its algorithmic
    bytes.  HIP events on the launch stream bracket blocks of back-to-back
    calls (the host issues a call in a fraction of its GPU time, so the queue
    never drains): a block's time per call is the kernel's duration plus the
    launch gap, without the host latency that per-call event pairs add."""
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(st.B, Hq, st.D, generator=g, device=device) * st.D ** -0.5
    out = torch.empty_like(q)
    settle_clocks(lambda: st.attention(q, out=out))
    per_block = max(1, iters // blocks)
    ms = []
    for _ in range(blocks):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(per_block):
            st.attention(q, out=out)
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1) / per_block)
    ms.sort()
    avg = sum(ms) / len(ms)
    nbytes = attn_bytes(st.B, Hq, st.H, st.D, st.quantized_tokens, st.res_len, st.G, st.Gv)
    return {"avg_us": avg * 1e3, "median_us": ms[len(ms) // 2] * 1e3, "bytes": nbytes,
            "gbs": nbytes / (avg * 1e-3) / 1e9, "Tq": st.quantized_tokens, "Tr": st.res_len}


def decode_loop(st, Hq, steps, warmup, R, seed, device):
    """The timed decode loop: fused append + attention, then the flush when
    the window reaches R."""
    import torch
    B, Hkv, D, G, Gv = st.B, st.H, st.D, st.G, st.Gv
    n = steps + warmup
    g = torch.Generator(device=device).manual_seed(seed)
    k_new, v_new = synth_kv(B, Hkv, n, D, seed + 1, device)
    q_all = torch.randn(n, B, Hq, D, generator=g, device=device) * D ** -0.5
    out = torch.empty(B, Hq, D, device=device)

    def step(i):
        # the new token is written by the attention launch itself; the G
        # oldest residual tokens are quantised once the window holds R
        st.stage_token(k_new[:, :, i:i + 1], v_new[:, :, i:i + 1])
        nb = append_bytes(B, Hkv, D)
        nb += attn_bytes(B, Hq, Hkv, D, st.quantized_tokens, st.res_len, G, Gv)
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
    wall0 = time.perf_counter()
    t0.record()
    for i in range(warmup, n):
        nb, fl = step(i)
        total_bytes += nb
        total_flushes += fl
    t1.record()
    submit = time.perf_counter() - wall0     # host time to issue the K steps
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1)
    return {"ms": ms, "wall_s": wall, "submit_s": submit, "bytes": total_bytes,
            "flushes": total_flushes,
            "gbs": total_bytes / (ms * 1e-3) / 1e9, "ms_per_step": ms / steps}


def quantize_bench(device, iters=10):
    """Config 2: keys [8,32,128,4096] (G=32 along tokens) + values
    [8,32,4096,128] (G=32 along D); Mtokens/s where a token is one (b, t)
    position with all 32 heads of K and V."""
    import torch
    from intel_kivi_hybrid_amd import _C
    B, H, D, S, G = 8, 32, 128, 4096, 32
    N = B * H * D * S
    k, v = synth_kv(B, H, S, D, 1236, device)
    kt = k.transpose(2, 3).contiguous()
    del k
    kp = torch.empty(N // 4, dtype=torch.uint8, device=device)
    ks = torch.empty(N // G, device=device)
    kz = torch.empty(N // G, device=device)
    vp, vs, vz = torch.empty_like(kp), torch.empty_like(ks), torch.empty_like(kz)

    def one():
        _C.quantize_keys_async(kt, kp, ks, kz, G)
        _C.quantize_values_async(v, vp, vs, vz, D, G)

    for _ in range(2):
        one()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        one()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / iters
    nbytes = 2 * quant_bytes(N, G)
    tokens = B * S
    res = {"us_per_pair": us, "gbs": nbytes / (us * 1e-6) / 1e9,
           "mtokens_s": tokens / us, "bytes": nbytes, "tokens": tokens}
    # round-trip error / scale (reported, not gated)
    rt = torch.empty_like(v)
    _C.quant_dequant_roundtrip_values(v, rt, D, G)
    err = (rt - v).abs().reshape(-1, G).amax(dim=1)
    res["max_err_over_scale"] = float((err / vs).max())
    return res


def prefill_bench(device, iters=20):
    """Batched prefill flush: a 4096-token prompt of config 2's shape
    (B=8, 32 kv heads, D=128) appended to an empty PackedKVStore (R=128,
    G=32), which quantises its 125 owed chunks per (b, head) in one launch
    reading the [B,H,T,D] K/V in place; fp32 and bf16 inputs.  Algorithmic
    bytes: the flushed tokens' K/V read once plus the codes, scales and
    zeros written; Mtokens/s counts (b, t) positions with all heads of K and
    V."""
    import torch
    from intel_kivi_hybrid_amd.store import PackedKVStore
    B, H, T, D, G, R = 8, 32, 4096, 128, 32, 128
    k, v = synth_kv(B, H, T, D, 1237, device)
    out = {}
    for name, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        kk, vv = k.to(dt), v.to(dt)
        st = PackedKVStore(B, H, D, G, R, device, chunk_capacity=T // G + 1)

        def one():
            st.reset()
            st.extend(kk, vv, flush_at=R)

        settle_clocks(one)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            one()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / iters
        n_tok = st.n_chunks * G
        nbytes = (2 * B * H * n_tok * D * kk.element_size()       # K/V read
                  + 2 * B * H * n_tok * D // 4                     # codes
                  + B * H * st.n_chunks * D * 8                    # key scales + zeros
                  + B * H * n_tok * (D // G) * 8)                  # value scales + zeros
        out[name] = {"us": round(us, 1), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "mtokens_s": round(B * n_tok / us, 1), "chunks": st.n_chunks,
                     "bytes": nbytes}
        del st, kk, vv
    return out


# --------------------------------------------------------------------------
# CPU baselines (the reference's CPU path, restated; test infrastructure)
# --------------------------------------------------------------------------
def cpu_attention_baseline(B, Hq, Hkv, D, T, R, G, Gv, budget_s=10.0):
    """What the reference does per decode step on the CPU: HF-style fp32
    attention (repeat_kv, QK^T*scale, softmax, PV) over the dequantised
    history + fp32 residual served by get_full_cache()
    (src/kivi_sycl/cache/manager.py:251-290).  Timed on a sample of the batch
    with all host threads; reported in the same algorithmic-bytes unit."""
    import torch
    from oracle import codec  # noqa: F401  (the oracle codec builds the history below)
    n_flush = (T - R) // G + 1
    Tq, Tr = n_flush * G, T - n_flush * G
    nb = max(1, min(B, 4))
    g = torch.Generator().manual_seed(7)
    k = torch.randn(nb, Hkv, T, D, generator=g)
    v = torch.randn(nb, Hkv, T, D, generator=g)
    # the served history is the mirror round-trip of each flushed chunk
    kh = k[:, :, :Tq].reshape(nb, Hkv, Tq // G, G, D).transpose(3, 4).contiguous()
    kh = torch.from_numpy(codec.roundtrip_groups(kh.numpy(), G).reshape(kh.shape))
    kh = kh.transpose(3, 4).reshape(nb, Hkv, Tq, D)
    vh = torch.from_numpy(codec.roundtrip_groups(v[:, :, :Tq].contiguous().numpy(), Gv)
                          .reshape(nb, Hkv, Tq, D))
    K = torch.cat([kh, k[:, :, Tq:]], dim=2)
    V = torch.cat([vh, v[:, :, Tq:]], dim=2)
    q = torch.randn(nb, Hq, 1, D, generator=g) * D ** -0.5
    rep = Hq // Hkv

    def step():
        Kx = K[:, :, None].expand(nb, Hkv, rep, T, D).reshape(nb, Hq, T, D)
        Vx = V[:, :, None].expand(nb, Hkv, rep, T, D).reshape(nb, Hq, T, D)
        w = torch.matmul(q, Kx.transpose(-1, -2)) * D ** -0.5
        w = torch.softmax(w, dim=-1)
        return torch.matmul(w, Vx)

    step()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s and n < 10000:
        step()
        n += 1
    dt = (time.perf_counter() - t0) / n
    nbytes = attn_bytes(nb, Hq, Hkv, D, Tq, Tr, G, Gv)
    return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{nb} of {B} sequences x {Hkv} kv heads, context {T} (Tq={Tq}, Tr={Tr}), "
                      f"{n} steps in {n * dt:.1f}s; torch fp32 attention over the dequantised "
                      f"history as the reference's HF model computes it on the CPU"}


def cpu_quantize_baseline(budget_s=8.0):
    """The C oracle (one group per iteration, OpenMP over groups, the
    reference kernels' loop structure) on 1/8 of config 2."""
    import numpy as np
    from oracle import codec
    B, H, D, S, G = 1, 32, 128, 4096, 32
    rng = np.random.default_rng(0)
    k = rng.standard_normal((B, H, D, S), dtype=np.float32)
    v = rng.standard_normal((B, H, S, D), dtype=np.float32)
    codec.quantize_groups(k, G)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s and n < 1000:
        codec.quantize_groups(k, G)
        codec.quantize_groups(v, G)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return {"value": B * S / dt / 1e6, "unit": "Mtokens/s", "cores": codec.num_threads(),
            "kind": "port",
            "sample": f"keys [1,32,128,4096] + values [1,32,4096,128] (1/8 of config 2), "
                      f"{n} passes in {n * dt:.1f}s"}


# --------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--attn-iters", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["config4", "attention", "quantize", "prefill", "copy"],
                    default=None,
                    help="run one workload (for profiling); 'copy' is a plain 512 MiB device "
                         "copy used to calibrate the FETCH_SIZE / WRITE_SIZE counters")
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

    if args.only == "copy":
        n = 512 << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(7)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy: {n} bytes read and {n} bytes written per launch, 5 launches")
        return

    if args.only == "prefill":
        for name, r in prefill_bench(dev).items():
            log(f"[bench] prefill flush ({name}): {r}")
        return
    if args.only == "quantize":
        qb = quantize_bench(dev)
        log(f"[bench] config2 quantize K+V: {qb['us_per_pair']:.1f} us, {qb['gbs']:.0f} GB/s, "
            f"{qb['mtokens_s']:.1f} Mtokens/s")
        return

    # ---- config 4: the headline decode loop -------------------------------
    B, Hq, Hkv, D, T, R, G = 64, 32, 8, 128, 8192, 128, 32
    log(f"[bench] config4 store: B={B} Hq={Hq} Hkv={Hkv} D={D} T={T} R={R} G={G}")
    st = build_store(B, Hkv, D, G, G, R, T, 1234 + 4, dev,
                     extra_chunks=(args.steps + args.warmup) // G + 2)
    torch.cuda.synchronize()
    if args.only == "attention":
        r = time_attention(st, Hq, args.attn_iters, 5, dev)
        log(f"[bench] attention only: {r}")
        return
    attn4 = time_attention(st, Hq, args.attn_iters, 5, dev)
    log(f"[bench] config4 attention: {attn4['avg_us']:.1f} us, {attn4['gbs']:.0f} GB/s")
    loop = decode_loop(st, Hq, args.steps, args.warmup, R, 99, dev)
    log(f"[bench] config4 decode loop: {loop['ms_per_step'] * 1e3:.1f} us/step, "
        f"{loop['gbs']:.0f} GB/s, {loop['flushes']} flushes (host issues a step in "
        f"{loop['submit_s'] / args.steps * 1e6:.1f} us)")
    del st
    torch.cuda.empty_cache()
    if args.only == "config4":
        return

    extra = {}
    if args.only is None:
        # ---- config 3 (MHA) and config 5 (long context, Gv=128) ------------
        st3 = build_store(16, 32, 128, 32, 32, 128, 4096 + 128, 1234 + 3, dev)
        a3 = time_attention(st3, 32, args.attn_iters, 6, dev)
        log(f"[bench] config3 attention: {a3['avg_us']:.1f} us, {a3['gbs']:.0f} GB/s "
            f"(Tq={a3['Tq']}, Tr={a3['Tr']})")
        del st3
        torch.cuda.empty_cache()
        st5 = build_store(4, 8, 128, 32, 128, 128, 131072 + 128, 1234 + 5, dev)
        a5 = time_attention(st5, 32, args.attn_iters, 7, dev)
        log(f"[bench] config5 attention: {a5['avg_us']:.1f} us, {a5['gbs']:.0f} GB/s "
            f"(Tq={a5['Tq']}, Tr={a5['Tr']})")
        del st5
        torch.cuda.empty_cache()
        extra["attention_config3"] = {k: a3[k] for k in ("avg_us", "gbs", "Tq", "Tr")}
        extra["attention_config5"] = {k: a5[k] for k in ("avg_us", "gbs", "Tq", "Tr")}

    qb = quantize_bench(dev)
    log(f"[bench] config2 quantize K+V: {qb['us_per_pair']:.1f} us, {qb['gbs']:.0f} GB/s, "
        f"{qb['mtokens_s']:.1f} Mtokens/s")
    if args.only is None:
        pf = prefill_bench(dev)
        for name, r in pf.items():
            log(f"[bench] prefill flush ({name} K/V, 4096-token prompt, B=8, 32 heads): "
                f"{r['us']:.1f} us, {r['gbs']:.0f} GB/s, {r['mtokens_s']:.1f} Mtokens/s")
        extra["prefill_flush"] = pf

    cpu = cpu_q = None
    if not args.no_cpu_baseline:
        cpu = cpu_attention_baseline(B, Hq, Hkv, D, T, R, G, G)
        log(f"[bench] cpu baseline attention: {cpu}")
        cpu_q = cpu_quantize_baseline()
        log(f"[bench] cpu baseline quantize: {cpu_q}")

    line = {
        "metric": "packed-KV decode attention GB/s (% HBM peak) + quantize Mtokens/s, 1 GPU",
        "value": round(loop["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(loop["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded N(0,1) K/V with channel/token outliers, made on the GPU)",
        "config": {"workload": "config4 Llama-3-8B GQA packed-KV decode loop",
                   "batch": B, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D,
                   "context": T, "residual": R, "group_size": G,
                   "step": "attention with the new token appended in the same launch + flush when residual >= R"},
        "pct_hbm_peak": round(100 * loop["gbs"] / HBM_PEAK_GBS, 2),
        "quantize_mtokens_s": round(qb["mtokens_s"], 2),
        "quantize_gbs": round(qb["gbs"], 1),
        "quantize_config": "config2 keys [8,32,128,4096] G=32 + values [8,32,4096,128] G=32",
        "quantize_max_err_over_scale": round(qb["max_err_over_scale"], 4),
        "roofline": {"bound": "hbm", "achieved": round(attn4["gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(attn4["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": ATTN4_TRAFFIC_BYTES if attn4["bytes"] == ATTN4_ALGO_BYTES else None,
                     "kernel": "packed decode attention (config 4, one call)",
                     "avg_us": round(attn4["avg_us"], 2), "bytes_per_launch": attn4["bytes"]},
        "cpu_baseline": cpu,
        "cpu_baseline_quantize": cpu_q,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
