"""Benchmark of the per-layer attention step on one MI355X.

Workload: the V1 mixed ragged batch of Qwen3-4B attention (32 query heads,
8 kv heads, head_dim 128, 256-token pages): 24 decode rows with contexts drawn
uniform in [256, 4096] (seed 3) plus two 512-token prefill chunks with cached
prefixes 0 and 1024, 1048 new tokens, 512-page pool.  One step = the
slot-mapped KV write of the 1048 new tokens + the ragged attention, as
forward_mixed runs them: with a bf16 pool ONE launch that also writes the new
K/V (the new tokens are read from their rows), with an E4M3FN pool the store
kernel and then one attention launch.

* value: whole-step throughput in tokens/s (1048 tokens per step), from HIP
  graph replays of 4 consecutive steps that rotate over 4 copies of the pool
  (4 x 512 MiB) so that no step finds its KV in the 256 MB Infinity Cache.
* roofline: the fused attention kernel against HBM bandwidth; achieved =
  algorithmic bytes per launch (decode KV bytes + prefill K/V + q + out, and
  with a bf16 pool the folded KV write: new rows read + slots written) /
  average launch duration (HIP events around the launch on its stream; a
  spin kernel queued ahead keeps host launch latency out of the interval, and
  consecutive launches rotate over the 4 pool copies so the KV is read from
  HBM, not from the Infinity Cache).  roofline_decode / roofline_prefill
  time the split launches (decode rows only against HBM, prefill rows only
  against bf16 MFMA peak), the mode that mirrors the reference's per-phase
  flash-attn calls.
* roofline_qk_norm_rope_store: the step before attention (q/k RMSNorm, RoPE
  and the KV write fused into one launch) on the same new tokens, against HBM.
* roofline_lm_head_argmax: the step after the model (LM head + greedy argmax
  fused, Qwen3-4B head 151936 x 2560 bf16) on the step's 26 sampled rows,
  against HBM (the weight read dominates).
* cpu_baseline: the CPU oracle (fp32 PyTorch on the host cores) on the same
  step.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "slo-aware-llm-serving-engine_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
# spin kernel queued ahead of each event-timed launch (about 0.4 ms): longer than
# the host time of any launch call here, so the GPU never waits for the host
# inside an event pair
SPIN_CYCLES = 1_000_000
METRIC = "mixed-step attn tokens/s; decode KV HBM GB/s (% of peak); prefill MFMA util"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kv", choices=["bf16", "fp8"], default="bf16")
    ap.add_argument("--events", type=int, default=100, help="event-timed launches per mode")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile", choices=["fused", "decode", "prefill", "qk", "lm_head"], default=None,
                    help="only launch this attention phase or kernel (for rocprofv3 counter runs), plus one "
                         "256 MiB device copy whose counters calibrate FETCH_SIZE/WRITE_SIZE")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the attention path runs at TP=1 and this build has no multi-GPU path).", file=sys.stderr)
        sys.exit(2)
    import torch
    from slo_attn import (_lib, forward_mixed, lm_head_argmax, qk_norm_rope_store, reserve_workspace, rope_cos_sin,
                          store_kvcache, workloads)
    from slo_attn.ops import paged_attention
    from types import SimpleNamespace

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    w = workloads.config(3)
    fp8 = args.kv == "fp8"
    dev = workloads.to_device(w, device)
    meta, slots = dev["meta"], dev["slot_mapping"]
    q, k, v = dev["q"], dev["k"], dev["v"]
    ctx = SimpleNamespace(mixed=meta, slot_mapping=slots)
    nsets = 4
    pools = []
    base_k, base_v = w.k_cache.to(device), w.v_cache.to(device)
    for _ in range(nsets):
        if fp8:
            nblk, bs, hkv, d = base_k.shape
            kc = torch.empty(nblk, bs, hkv, d, dtype=torch.uint8, device=device)
            vc = torch.empty_like(kc)
            ks = torch.empty(nblk, bs, hkv, dtype=torch.float32, device=device)
            vs = torch.empty_like(ks)
            allslots = torch.arange(nblk * bs, dtype=torch.int32, device=device)
            store_kvcache(base_k.view(-1, hkv, d), base_v.view(-1, hkv, d), kc, vc, allslots, ks, vs)
            pools.append((kc, vc, ks, vs))
        else:
            pools.append((base_k.clone(), base_v.clone(), None, None))
    del base_k, base_v
    torch.cuda.synchronize()
    reserve_workspace(device, w.num_decode, max(len(t) for t in w.decode_tables) * w.block_size, 32, 8, 128)

    def step(i, phases=_lib.PHASE_ALL):
        kc, vc, ks, vs = pools[i % nsets]
        return forward_mixed(q, k, v, kc, vc, ctx, w.scale, store_kvcache, ks, vs, phases=phases)

    # The step's own launch: with a bf16 pool forward_mixed folds the KV write
    # into the attention launch (fold=True); the split per-phase launches run
    # without it, as the reference's per-phase calls do.
    def attn_only(i, phases, fold=False):
        kc, vc, ks, vs = pools[i % nsets]
        store = dict(store_slot_mapping=slots, new_k=k, new_v=v) if fold else {}
        return paged_attention(
            q, kc, vc, w.scale, num_kv_heads=8, k_scale=ks, v_scale=vs, num_decode=meta.num_decode,
            decode_lens=meta.decode_lens, decode_tables=meta.decode_tables,
            num_prefill=meta.prefill_cu_q.numel() - 1, prefill_cu_q=meta.prefill_cu_q,
            prefill_cu_k=meta.prefill_cu_k, max_q=meta.max_q, max_k=meta.max_k,
            prefill_tables=meta.prefill_tables, phases=phases, out=out_buf, **store)

    hq, hkv, d = 32, 8, 128
    elem = 1.0 if fp8 else 2.0
    scale_b = 4 if fp8 else 0
    tokens = w.num_tokens

    # ---- the step before attention: fused q/k RMSNorm + RoPE + KV write of the
    # same new tokens from a synthetic QKV projection output [tokens, 48*128]
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(tokens, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16).to(device)
    positions = [L - 1 for L in w.decode_lens]
    for n, pfx in zip(w.prefill_q, w.prefill_prefix):
        positions += list(range(pfx, pfx + n))
    positions = torch.tensor(positions, dtype=torch.int64, device=device)
    qn_w = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(device)
    kn_w = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(device)
    cos_sin = rope_cos_sin(d, 40960, 1e6, device)

    def qk_launch(i):
        kc, vc, ks, vs = pools[i % nsets]
        qk_norm_rope_store(qkv, positions, qn_w, kn_w, 1e-6, cos_sin, hq, hkv, kc, vc, slots, ks, vs)

    # read the QKV row, positions and one cos/sin row per token; write q, k and the K/V pool entries
    qk_bytes = tokens * ((hq + 2 * hkv) * d * 2 + 8 + d * 4 + 4 + (hq + hkv) * d * 2 + 2 * hkv * (d * elem + scale_b))

    # ---- the step after the model: LM head + greedy argmax on the step's sampled
    # rows (every decode row and the last token of each prefill chunk) over the
    # Qwen3-4B head [151936, 2560]; two weight copies alternate so each launch
    # streams its 778 MB weight from HBM
    vocab, hidden = 151936, 2560
    sample_rows = w.num_decode + len(w.prefill_q)
    heads = []
    if args.profile in (None, "lm_head"):
        gd = torch.Generator(device=device).manual_seed(6)
        heads = [torch.empty(vocab, hidden, dtype=torch.bfloat16, device=device).normal_(0, 0.02, generator=gd)
                 for _ in range(2)]
        hid = torch.empty(sample_rows, hidden, dtype=torch.bfloat16, device=device).normal_(0, 1, generator=gd)

    def lm_launch(i):
        lm_head_argmax(hid, heads[i % 2])

    # weight + sampled hidden rows read, one int64 token per row written
    lm_bytes = vocab * hidden * 2 + sample_rows * hidden * 2 + sample_rows * 8

    def timed(fn, warmup=None, n=None):
        """Average HIP-event duration of fn(i) on the current stream; a spin kernel
        queued ahead keeps host launch latency out of the interval."""
        warmup = args.warmup if warmup is None else warmup
        times = []
        for i in range(warmup + (args.events if n is None else n)):
            torch.cuda._sleep(SPIN_CYCLES)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            fn(i)
            e1.record()
            e1.synchronize()
            if i >= warmup:
                times.append(e0.elapsed_time(e1) * 1e3)
        return statistics.mean(times)

    out_buf = torch.empty_like(q)
    if args.profile:
        launch = {"fused": lambda i: attn_only(i, _lib.PHASE_ALL, not fp8), "decode": lambda i: attn_only(i, _lib.PHASE_DECODE),
                  "prefill": lambda i: attn_only(i, _lib.PHASE_PREFILL), "qk": qk_launch,
                  "lm_head": lm_launch}[args.profile]
        src = torch.empty(256 << 20, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)  # calibration: 256 MiB read + 256 MiB written
        avg = timed(launch, args.warmup, args.events)
        print(json.dumps({"profile": args.profile, "launches": args.warmup + args.events,
                          "avg_launch_us": round(avg, 2)}))
        return
    for i in range(max(args.warmup, 4)):
        step(i)
    torch.cuda.synchronize()

    # ---- whole-step throughput from graph replays (4 steps per replay)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(nsets):
            step(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for i in range(nsets):
            step(i)
    for _ in range(max(1, args.warmup // nsets)):
        graph.replay()
    torch.cuda.synchronize()
    # Untimed settling: keep the GPU busy with the same replays for about
    # 0.3 s, so the timed steps run at the clocks a serving loop sees (the
    # first tens of milliseconds after an idle period ran ~5% slower here).
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < 0.3:
        for _ in range(20):
            graph.replay()
        torch.cuda.synchronize()
    replays = max(1, (args.steps + nsets - 1) // nsets)
    steps = replays * nsets
    t0 = time.perf_counter()
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / steps
    value = tokens * steps / elapsed

    # ---- per-launch kernel durations (HIP events on the launch stream, cold cache)
    def launch_times(phases, fold=False):
        stream = torch.cuda.current_stream()
        times = []
        for i in range(args.events + args.warmup):
            torch.cuda._sleep(SPIN_CYCLES)  # GPU-side backlog: the events bracket only the launch
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            attn_only(i, phases, fold)
            e1.record(stream)
            e1.synchronize()
            if i >= args.warmup:
                times.append(e0.elapsed_time(e1) * 1e3)  # us
        return statistics.mean(times), statistics.median(times)

    t_fused, t_fused_med = launch_times(_lib.PHASE_ALL, not fp8)
    t_dec, t_dec_med = launch_times(_lib.PHASE_DECODE)
    t_pre, t_pre_med = launch_times(_lib.PHASE_PREFILL)

    dec_bytes = w.decode_kv_bytes(elem, scale_b)
    pre_kv_tokens = sum(n + p for n, p in zip(w.prefill_q, w.prefill_prefix))
    pre_bytes = pre_kv_tokens * hkv * (2 * d * elem + 2 * scale_b)
    qo_bytes = 2 * tokens * hq * d * 2
    # the KV write folded into the bf16 launch: new K/V rows read, pool slots written
    store_bytes = 0 if fp8 else 2 * tokens * hkv * d * 2 * 2
    fused_bytes = dec_bytes + pre_bytes + qo_bytes + store_bytes
    flops = w.prefill_flops()
    fused_gbs = fused_bytes / (t_fused * 1e-6) / 1e9
    dec_gbs = (dec_bytes + 2 * w.num_decode * hq * d * 2) / (t_dec * 1e-6) / 1e9
    pre_tflops = flops / (t_pre * 1e-6) / 1e12

    t_qk = timed(qk_launch)
    qk_gbs = qk_bytes / (t_qk * 1e-6) / 1e9
    t_lm = timed(lm_launch)
    lm_gbs = lm_bytes / (t_lm * 1e-6) / 1e9
    # the reference's path on the same inputs: compute_logits (F.linear) then argmax
    t_lm_torch = timed(lambda i: torch.nn.functional.linear(hid, heads[i % 2]).argmax(dim=-1))
    del heads

    # HBM bytes per fused launch measured by rocprofv3 (FETCH_SIZE + WRITE_SIZE,
    # calibrated against a 256 MiB copy) for this kernel, kept under profiles/.
    measured = {}
    tpath = os.path.join(ROOT, "profiles", "traffic_mixed_24decode_2x512chunk.json")
    if not fp8 and os.path.exists(tpath):
        with open(tpath) as fh:
            measured = json.load(fh)

    def traffic(kernel):
        return round(measured[kernel]["traffic_mb"] * 1e6) if kernel in measured else None

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(w, fp8)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1), unit-RMS q/k)",
        "config": {
            "workload": w.name, "decode_rows": w.num_decode, "decode_context_sum": sum(w.decode_lens),
            "prefill_chunks": w.prefill_q, "prefill_prefixes": w.prefill_prefix, "new_tokens": tokens,
            "heads": [hq, hkv, d], "block_size": w.block_size, "kv_cache": args.kv,
            "step": ("store_kvcache + one fused ragged attention launch" if fp8 else
                     "one fused ragged attention launch with the KV write folded in (forward_mixed)"),
            "pool_copies_rotated": nsets,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(fused_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(fused_gbs / HBM_PEAK_GBS, 4), "traffic": traffic("fused"),
            "kernel": "paged_attention_kernel (fused decode+prefill" + ("" if fp8 else ", KV write folded in") + ")",
            "algorithmic_bytes_per_launch": fused_bytes, "avg_launch_us": round(t_fused, 2),
            "median_launch_us": round(t_fused_med, 2),
        },
        "roofline_decode": {
            "bound": "hbm", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dec_gbs / HBM_PEAK_GBS, 4), "decode_kv_bytes": dec_bytes,
            "avg_launch_us": round(t_dec, 2), "median_launch_us": round(t_dec_med, 2),
        },
        "roofline_prefill": {
            "bound": "mfma", "achieved": round(pre_tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(pre_tflops / BF16_PEAK_TFLOPS, 4), "flops": flops,
            "avg_launch_us": round(t_pre, 2), "median_launch_us": round(t_pre_med, 2),
        },
        "split_step_us": round(t_dec + t_pre, 2),
        "roofline_qk_norm_rope_store": {
            "bound": "hbm", "achieved": round(qk_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(qk_gbs / HBM_PEAK_GBS, 4), "traffic": traffic("qk"), "kernel": "qk_norm_rope_store_kernel",
            "algorithmic_bytes_per_launch": qk_bytes, "avg_launch_us": round(t_qk, 2),
            "tokens": tokens,
        },
        "roofline_lm_head_argmax": {
            "bound": "hbm", "achieved": round(lm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(lm_gbs / HBM_PEAK_GBS, 4), "traffic": traffic("lm_head"), "kernel": "lm_head_argmax_kernel",
            "algorithmic_bytes_per_launch": lm_bytes, "avg_launch_us": round(t_lm, 2),
            "rows": sample_rows, "vocab": vocab, "hidden": hidden,
            "torch_linear_argmax_us": round(t_lm_torch, 2),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def cpu_baseline(w, fp8):
    """The CPU oracle (fp32 torch on the host cores) on the same step."""
    import numpy as np
    import torch
    from oracle import attention as oatt
    from oracle import fp8 as ofp8
    from oracle import kvstore
    from slo_attn.workloads import padded_tables

    meta = {
        "num_decode": w.num_decode, "num_prefill_tokens": sum(w.prefill_q), "decode_lens": w.decode_lens,
        "decode_tables": padded_tables(w.decode_tables), "prefill_cu_q": w.cu_q, "prefill_cu_k": w.cu_k,
        "prefill_tables": padded_tables(w.prefill_tables), "prefill_has_history": w.has_history,
    }
    kc = w.k_cache.clone()
    vc = w.v_cache.clone()
    if fp8:
        kcodes, kscale = ofp8.quantize_kv(kc.float().numpy())
        vcodes, vscale = ofp8.quantize_kv(vc.float().numpy())

    def run():
        if fp8:
            kvstore.store_kvcache_fp8(w.k.float().numpy(), w.v.float().numpy(), kcodes, vcodes, kscale, vscale,
                                      w.slot_mapping)
            kf = torch.from_numpy(ofp8.dequantize_kv(kcodes, kscale))
            vf = torch.from_numpy(ofp8.dequantize_kv(vcodes, vscale))
        else:
            kvstore.store_kvcache(w.k.view(torch.int16).numpy(), w.v.view(torch.int16).numpy(),
                                  kc.view(torch.int16).numpy(), vc.view(torch.int16).numpy(), w.slot_mapping)
            kf, vf = kc, vc
        return oatt.mixed(w.q.float(), w.k.float(), w.v.float(), kf, vf, meta, w.scale)

    run()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(w.num_tokens / t, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"full step ({w.num_tokens} tokens), median of 3 after 1 warm-up, "
                                      f"{t * 1e3:.1f} ms per step"}


if __name__ == "__main__":
    main()
