"""Benchmark of the per-layer attention step on one MI355X.

Workload: the V1 mixed ragged batch of Qwen3-4B attention (32 query heads,
8 kv heads, head_dim 128, 256-token pages): 24 decode rows with contexts drawn
uniform in [256, 4096] (seed 3) plus two 512-token prefill chunks with cached
prefixes 0 and 1024, 1048 new tokens, 512-page pool.  One step = the
slot-mapped KV write of the 1048 new tokens + the ragged attention, as
forward_mixed runs them: with a bf16 pool ONE launch that also writes the new
K/V (the new tokens are read from their rows), with an E4M3FN pool the store
kernel and then one attention launch.  (Steps without decode rows, the
prefill-only workloads of --configs, run the store kernel and then the
attention launch on either pool.)

Every time below comes from HIP-graph replays: a graph holds back-to-back
launches that rotate over 4 copies of the pool (4 x 512 MiB bf16), so no
launch finds its KV in the 256 MB Infinity Cache, after an untimed settling
phase (~0.3 s of the same replays, so the timed ones run at the clocks a
serving loop sees).  Per-launch times are HIP events on the replay stream
around the timed replays / launches, the ~1 us gap between back-to-back
kernels included; the whole-step throughput uses the host clock between two
device synchronisations.

* value: whole-step throughput in tokens/s (1048 tokens per step) over the
  --steps timed steps; ms_per_step is the same measurement.
* roofline: the step's attention launch (bf16 pool, KV write folded in)
  against HBM bandwidth: achieved = algorithmic bytes per launch (cached K/V
  read: decode contexts and prefill prefixes; each new token's bf16 K/V row
  read once and its pool slot written once; q read and out written) / its
  per-launch time.  roofline_decode / roofline_prefill time the
  split launches (decode rows only against HBM, prefill rows only against bf16
  MFMA peak), the mode that mirrors the reference's per-phase flash-attn calls;
  roofline_prefill carries the MFMA-busy fraction that rocprofv3 counters gave
  for that launch (profiles/counters_paged_attention.json).
* roofline_fp8: the same step and split launches on an E4M3FN pool (codes +
  per-(token, kv head) fp32 scales).
* tp2_rank: the step at one TP=2 rank's head shape (16 query / 4 kv heads, the
  same rows and tables).
* roofline_qk_norm_rope_store: the step before attention (q/k RMSNorm, RoPE
  and the KV write fused into one launch) on the same new tokens, against HBM.
* roofline_lm_head_argmax: the step after the model (LM head + greedy argmax
  fused, Qwen3-4B head 151936 x 2560 bf16) on the step's 26 sampled rows,
  against HBM (the weight read dominates).
* roofline_decode.read_ceiling: what a plain read of the same byte count
  achieves on this GPU (read_ceiling, built from read_ceiling.hip next to
  this file by __graft_entry__.build(), run as a child process: one-pass
  streams into VGPRs and through LDS-DMA with the default and the
  non-temporal cache policy, the last the decode kernels' route, and the
  decode kernels' access pattern: one kv head's 256-byte slice of each 2 KiB
  pool row), and the decode launch's rate as a fraction of the non-temporal
  LDS-DMA stream and of the head-slice read with the kv heads of a row range
  on different XCDs (the mapping the config-3 decode launch takes).
* Pool copies: enough are rotated that the launches read at least twice the
  MI355X Infinity Cache (256 MiB) between two visits of one copy, so the KV
  bytes come from HBM (4 copies for the config-3 step, 17 for config 0).
* cpu_baseline: the CPU oracle (fp32 PyTorch on the host cores) on the same
  step, median of 5 runs after 1 warm-up.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "slo-aware-llm-serving-engine_amd"))
sys.path.insert(0, ROOT)

import workloads  # noqa: E402  (seeded synthetic inputs, next to this file)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "mixed-step attn tokens/s; decode KV HBM GB/s (% of peak); prefill MFMA util"
NSETS = 4            # pool copies rotated by consecutive launches (at least)
MALL_BYTES = 256 << 20  # MI355X Infinity Cache: rotated copies read at least twice this
SETTLE_S = 0.3       # untimed replays before each timed measurement
LAUNCH_TARGET = 1200  # launches per per-launch measurement


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=3, help="workload of --profile runs (0-4)")
    ap.add_argument("--kv", choices=["bf16", "fp8"], default="bf16", help="pool format of --profile runs")
    ap.add_argument("--events", type=int, default=100, help="launches of --profile runs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the step line: one JSON line per workload config 0-4 (step, decode and "
                         "prefill launches on both pool formats, and the CPU oracle's step time)")
    ap.add_argument("--profile", choices=["fused", "decode", "prefill", "qk", "lm_head"], default=None,
                    help="only launch this attention phase or kernel (eagerly, for rocprofv3 counter runs) on "
                         "--config / --kv, plus one 256 MiB device copy whose counters calibrate "
                         "FETCH_SIZE/WRITE_SIZE")
    return ap.parse_args()


class Step:
    """One attention workload on the GPU with `nsets` pool copies (bf16, or E4M3FN)."""

    def __init__(self, w, device, fp8):
        import torch
        from slo_attn import reserve_workspace, store_kvcache
        self.w, self.fp8, self.device = w, fp8, device
        dev = workloads.to_device(w, device)
        self.meta, self.slots = dev["meta"], dev["slot_mapping"]
        self.q, self.k, self.v = dev["q"], dev["k"], dev["v"]
        self.hq, self.hkv, self.d = w.q.shape[1], w.k.shape[1], w.q.shape[2]
        base_k, base_v = w.k_cache.to(device), w.v_cache.to(device)
        # Enough pool copies that the bytes the launches read from them between
        # two visits of one copy exceed twice the Infinity Cache, so every
        # launch reads its KV from HBM (4 at least; 4 when nothing is read
        # from the pool).
        row = self.hkv * (2 * self.d * self.elem() + 2 * self.scale_bytes())
        read = self.decode_bytes() + sum(w.prefill_prefix) * row
        self.nsets = NSETS if read == 0 else int(min(32, max(NSETS, math.ceil(2 * MALL_BYTES / read))))
        self.pools = []
        for _ in range(self.nsets):
            if fp8:
                nblk, bs, hkv, d = base_k.shape
                kc = torch.empty(nblk, bs, hkv, d, dtype=torch.uint8, device=device)
                vc = torch.empty_like(kc)
                ks = torch.empty(nblk, bs, hkv, dtype=torch.float32, device=device)
                vs = torch.empty_like(ks)
                allslots = torch.arange(nblk * bs, dtype=torch.int32, device=device)
                store_kvcache(base_k.view(-1, hkv, d), base_v.view(-1, hkv, d), kc, vc, allslots, ks, vs)
                self.pools.append((kc, vc, ks, vs))
            else:
                self.pools.append((base_k.clone(), base_v.clone(), None, None))
        del base_k, base_v
        torch.cuda.synchronize()
        reserve_workspace(device, w.num_decode, max([len(t) for t in w.decode_tables] + [1]) * w.block_size,
                          self.hq, self.hkv, self.d)
        self.out = torch.empty_like(self.q)
        from types import SimpleNamespace
        self.ctx = SimpleNamespace(mixed=self.meta, slot_mapping=self.slots)

    def step(self, i):
        """forward_mixed as the engine calls it (KV write folded in on a bf16 pool)."""
        from slo_attn import _lib, forward_mixed, store_kvcache
        kc, vc, ks, vs = self.pools[i % self.nsets]
        return forward_mixed(self.q, self.k, self.v, kc, vc, self.ctx, self.w.scale, store_kvcache, ks, vs,
                             phases=_lib.PHASE_ALL)

    def attn(self, i, phases, fold=False):
        """One attention launch without the KV write (or with it folded in)."""
        from slo_attn.ops import paged_attention
        kc, vc, ks, vs = self.pools[i % self.nsets]
        meta, w = self.meta, self.w
        store = dict(store_slot_mapping=self.slots, new_k=self.k, new_v=self.v) if fold else {}
        history = w.has_history or fold
        return paged_attention(
            self.q, kc, vc, w.scale, num_kv_heads=self.hkv, k_scale=ks, v_scale=vs, num_decode=meta.num_decode,
            decode_lens=meta.decode_lens, decode_tables=meta.decode_tables,
            num_prefill=(meta.prefill_cu_q.numel() - 1) if meta.prefill_cu_q is not None else 0,
            prefill_cu_q=meta.prefill_cu_q, prefill_cu_k=meta.prefill_cu_k, max_q=meta.max_q, max_k=meta.max_k,
            prefill_tables=meta.prefill_tables if history else None, k=None if history else self.k[w.num_decode:],
            v=None if history else self.v[w.num_decode:], phases=phases, out=self.out, **store)

    def time(self, fn):
        """graph_time over one launch per pool copy."""
        return graph_time(fn, n_per_graph=self.nsets)

    def elem(self):
        return 1.0 if self.fp8 else 2.0

    def scale_bytes(self):
        return 4 if self.fp8 else 0

    def decode_bytes(self):
        return self.w.decode_kv_bytes(self.elem(), self.scale_bytes())

    def step_bytes(self, fold):
        """Algorithmic bytes of one mixed launch: q read and out written, plus the
        pool K/V read (decode contexts, prefill prefixes and new rows).  With the KV
        write folded in, each new token's K/V counts once as read (its bf16 row of
        new_k/new_v) and once as written (its pool slot); the kernel's reads of it
        back from the pool add nothing."""
        w = self.w
        row = self.hkv * (2 * self.d * self.elem() + 2 * self.scale_bytes())
        qo = 2 * w.num_tokens * self.hq * self.d * 2
        if not fold:
            pre_tokens = sum(n + p for n, p in zip(w.prefill_q, w.prefill_prefix))
            return self.decode_bytes() + pre_tokens * row + qo
        cached = self.decode_bytes() - w.num_decode * row + sum(w.prefill_prefix) * row
        new = w.num_tokens * (2 * self.hkv * self.d * 2 + row)
        return cached + new + qo


def graph_time(fn, n_per_graph=NSETS, target=LAUNCH_TARGET, replays=None):
    """Average time per launch (us) of fn(i), i = 0..n_per_graph-1 captured back to back
    in one HIP graph: HIP events on the replay stream bracket the timed replays,
    which follow an untimed settling phase."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(n_per_graph):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n_per_graph):
            fn(i)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < SETTLE_S:
        for _ in range(10):
            graph.replay()
        torch.cuda.synchronize()
    n = replays if replays is not None else max(1, target // n_per_graph)
    stream = torch.cuda.current_stream()  # the replays' (and so the kernels') stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(n):
        graph.replay()
    e1.record(stream)
    e1.synchronize()
    dt_ms = e0.elapsed_time(e1)
    del graph
    return dt_ms * 1e3 / (n * n_per_graph), n * n_per_graph


def hbm(bytes_, us, **extra):
    gbs = bytes_ / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), **extra}


def read_ceiling(nbytes):
    """Achievable read rates for nbytes: the read_ceiling program built next to
    this file, run as a child process (None when it is not built or fails)."""
    exe = os.path.join(ROOT, "read_ceiling")
    if not os.path.exists(exe):
        return None
    try:
        res = subprocess.run([exe, str(int(nbytes))], capture_output=True, text=True, timeout=120)
        return json.loads(res.stdout.strip().splitlines()[-1]) if res.returncode == 0 else None
    except (subprocess.TimeoutExpired, ValueError, IndexError):
        return None


def sources_sha16():
    """sha256 (first 16 hex digits) of the HIP sources the library is built from,
    in name order: profiles record the value of the build they measured."""
    import hashlib
    csrc = os.path.join(ROOT, "slo-aware-llm-serving-engine_amd", "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h", ".cpp")):
            h.update(name.encode())
            with open(os.path.join(csrc, name), "rb") as fh:
                h.update(fh.read())
    return h.hexdigest()[:16]


def load_profile_json(name):
    path = os.path.join(ROOT, "profiles", name)
    if os.path.exists(path):
        with open(path) as fh:
            return json.load(fh)
    return {}


def profile_stamp(profile, name):
    """Which build a profile-sourced field comes from: the sources hash the profile
    recorded and whether it equals the current sources' (a field from another
    build is kept but marked)."""
    recorded = profile.get("meta", {}).get("sources_sha16")
    current = sources_sha16()
    return {"file": f"profiles/{name}", "sources_sha16": recorded, "current_sources_sha16": current,
            "matches_build": recorded == current}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the attention path runs at TP=1 and this build has no multi-GPU path).", file=sys.stderr)
        sys.exit(2)
    import torch
    from slo_attn import _lib, lm_head_argmax, qk_norm_rope_store, rope_cos_sin

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.profile:
        return profile(args, device)
    if args.configs:
        return config_table(args, device)

    w = workloads.config(3)
    st = Step(w, device, fp8=False)
    hq, hkv, d = st.hq, st.hkv, st.d
    tokens = w.num_tokens

    # ---- whole-step throughput: graph replays of one step per pool copy
    for i in range(max(args.warmup, st.nsets)):
        st.step(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(st.nsets):
            st.step(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for i in range(st.nsets):
            st.step(i)
    for _ in range(max(1, args.warmup // st.nsets)):
        graph.replay()
    torch.cuda.synchronize()
    t_settle = time.perf_counter()  # untimed settling replays (steady-state clocks)
    while time.perf_counter() - t_settle < SETTLE_S:
        for _ in range(20):
            graph.replay()
        torch.cuda.synchronize()
    replays = max(1, (args.steps + st.nsets - 1) // st.nsets)
    steps = replays * st.nsets
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    del graph
    ms_per_step = elapsed * 1e3 / steps
    value = tokens * steps / elapsed

    # ---- per-launch times (graph replays of back-to-back launches)
    t_fused, n_fused = st.time(lambda i: st.attn(i, _lib.PHASE_ALL, fold=True))
    t_dec, _ = st.time(lambda i: st.attn(i, _lib.PHASE_DECODE))
    t_pre, _ = st.time(lambda i: st.attn(i, _lib.PHASE_PREFILL))
    fused_bytes = st.step_bytes(fold=True)
    dec_bytes = st.decode_bytes()
    flops = w.prefill_flops()
    pre_tflops = flops / (t_pre * 1e-6) / 1e12

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
        kc, vc, ks, vs = st.pools[i % st.nsets]
        qk_norm_rope_store(qkv, positions, qn_w, kn_w, 1e-6, cos_sin, hq, hkv, kc, vc, st.slots, ks, vs)

    # QKV row, position, cos/sin row and slot read; q, k and the K/V pool entries written
    qk_bytes = tokens * ((hq + 2 * hkv) * d * 2 + 8 + d * 4 + 4 + (hq + hkv) * d * 2 + 2 * hkv * d * 2)
    t_qk, _ = st.time(qk_launch)

    # ---- the step after the model: LM head + greedy argmax on the step's sampled
    # rows over the Qwen3-4B head [151936, 2560]; two weight copies alternate so each
    # launch streams its 778 MB weight from HBM
    vocab, hidden = 151936, 2560
    sample_rows = w.num_decode + len(w.prefill_q)
    gd = torch.Generator(device=device).manual_seed(6)
    heads = [torch.empty(vocab, hidden, dtype=torch.bfloat16, device=device).normal_(0, 0.02, generator=gd)
             for _ in range(2)]
    hid = torch.empty(sample_rows, hidden, dtype=torch.bfloat16, device=device).normal_(0, 1, generator=gd)
    lm_head_argmax(hid, heads[0])
    lm_bytes = vocab * hidden * 2 + sample_rows * hidden * 2 + sample_rows * 8
    t_lm, _ = graph_time(lambda i: lm_head_argmax(hid, heads[i % 2]), n_per_graph=2, target=200)
    # the reference's path on the same inputs: compute_logits (F.linear) then argmax
    t_lm_torch, _ = graph_time(lambda i: torch.nn.functional.linear(hid, heads[i % 2]).argmax(dim=-1),
                               n_per_graph=2, target=200)
    nsets = st.nsets
    del heads, st
    torch.cuda.empty_cache()

    # ---- E4M3FN pool: the step (store kernel + attention launch) and the split launches
    st8 = Step(w, device, fp8=True)
    t8_step, _ = st8.time(st8.step)
    t8_fused, _ = st8.time(lambda i: st8.attn(i, _lib.PHASE_ALL))
    t8_dec, _ = st8.time(lambda i: st8.attn(i, _lib.PHASE_DECODE))
    t8_pre, _ = st8.time(lambda i: st8.attn(i, _lib.PHASE_PREFILL))
    fp8_dec_bytes = st8.decode_bytes()
    fp8_fused_bytes = st8.step_bytes(fold=False)
    del st8
    torch.cuda.empty_cache()

    # ---- one TP=2 rank's head shape (16 query / 4 kv heads), same rows and tables
    w2 = workloads.config(3, 16, 4)
    st2 = Step(w2, device, fp8=False)
    t2_fused, _ = st2.time(lambda i: st2.attn(i, _lib.PHASE_ALL, fold=True))
    t2_dec, _ = st2.time(lambda i: st2.attn(i, _lib.PHASE_DECODE))
    t2_bytes, t2_dec_bytes = st2.step_bytes(fold=True), st2.decode_bytes()
    del st2
    torch.cuda.empty_cache()

    traffic = load_profile_json("traffic_mixed_24decode_2x512chunk.json")
    all_counters = load_profile_json("counters_paged_attention.json")
    counters = all_counters.get("prefill_3", {})

    def traffic_of(kernel):
        return round(traffic[kernel]["traffic_mb"] * 1e6) if kernel in traffic and kernel != "meta" else None

    # ---- 16 short decode rows (64-1024 tokens): a pure decode step (forward_mixed,
    # KV write folded in) and the decode launch alone, both pool formats
    w0 = workloads.config(0)
    small = {"workload": w0.name, "decode_rows": w0.num_decode, "decode_context_sum": sum(w0.decode_lens)}
    for fp8 in (False, True):
        st0 = Step(w0, device, fp8=fp8)
        t0_step, _ = st0.time(st0.step)
        t0_dec, _ = st0.time(lambda i: st0.attn(i, _lib.PHASE_DECODE))
        small["e4m3fn" if fp8 else "bf16"] = {
            "step_us": round(t0_step, 2),
            "decode": hbm(st0.decode_bytes(), t0_dec, avg_launch_us=round(t0_dec, 2), decode_kv_bytes=st0.decode_bytes(),
                          traffic=traffic_of("decode0_fp8" if fp8 else "decode0"), kernel="decode_direct_kernel"),
        }
        del st0
        torch.cuda.empty_cache()

    ceiling = read_ceiling(dec_bytes)
    if ceiling:
        # The decode kernels stream K/V by non-temporal LDS-DMA.
        ceiling["decode_frac_of_lds_dma_stream"] = round(
            dec_bytes / (t_dec * 1e-6) / (ceiling.get("stream_lds_dma_nt_TBps", ceiling["stream_lds_dma_TBps"]) * 1e12), 4)
        if ceiling.get("head_slices_spread_TBps"):
            ceiling["decode_frac_of_head_slice_stream"] = round(
                dec_bytes / (t_dec * 1e-6) / (ceiling["head_slices_spread_TBps"] * 1e12), 4)
    cpu = None if args.no_cpu_baseline else cpu_baseline(w)
    timing = f"HIP-graph replays of {nsets} back-to-back launches over {nsets} pool copies; us per launch"
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
            "heads": [hq, hkv, d], "block_size": w.block_size, "kv_cache": "bf16",
            "step": "one fused ragged attention launch with the KV write folded in (forward_mixed)",
            "pool_copies_rotated": nsets,
        },
        "roofline": hbm(fused_bytes, t_fused, traffic=traffic_of("fused"),
                        kernel="paged_attention_kernel (fused decode+prefill, KV write folded in)",
                        algorithmic_bytes_per_launch=fused_bytes, avg_launch_us=round(t_fused, 2),
                        launches=n_fused, timing=timing),
        "roofline_decode": hbm(dec_bytes, t_dec, decode_kv_bytes=dec_bytes, traffic=traffic_of("decode"),
                               avg_launch_us=round(t_dec, 2), kernel="decode_direct_kernel",
                               read_ceiling=ceiling),
        "roofline_prefill": {
            "bound": "mfma", "achieved": round(pre_tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(pre_tflops / BF16_PEAK_TFLOPS, 4), "flops": flops, "avg_launch_us": round(t_pre, 2),
            "mfma_busy": counters.get("mfma_busy"), "traffic": traffic_of("prefill"),
        },
        "split_step_us": round(t_dec + t_pre, 2),
        "roofline_fp8": {
            "kv_cache": "e4m3fn codes + fp32 scale per (token, kv head)",
            "step_us": round(t8_step, 2), "step_tokens_per_s": round(tokens / (t8_step * 1e-6), 1),
            "fused": hbm(fp8_fused_bytes, t8_fused, avg_launch_us=round(t8_fused, 2),
                         algorithmic_bytes_per_launch=fp8_fused_bytes, traffic=traffic_of("fused_fp8")),
            "decode": hbm(fp8_dec_bytes, t8_dec, avg_launch_us=round(t8_dec, 2), decode_kv_bytes=fp8_dec_bytes,
                          traffic=traffic_of("decode_fp8")),
            "prefill": {"bound": "mfma", "avg_launch_us": round(t8_pre, 2),
                        "achieved": round(flops / (t8_pre * 1e-6) / 1e12, 1), "unit": "TFLOP/s",
                        "frac": round(flops / (t8_pre * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                        "mfma_busy": all_counters.get("prefill_3_fp8", {}).get("mfma_busy")},
        },
        "tp2_rank": {
            "heads": [16, 4, 128], "workload": w2.name,
            "fused": hbm(t2_bytes, t2_fused, avg_launch_us=round(t2_fused, 2), algorithmic_bytes_per_launch=t2_bytes),
            "decode": hbm(t2_dec_bytes, t2_dec, avg_launch_us=round(t2_dec, 2), decode_kv_bytes=t2_dec_bytes),
        },
        "decode_short_rows": small,
        "roofline_qk_norm_rope_store": hbm(qk_bytes, t_qk, traffic=traffic_of("qk"), kernel="qk_norm_rope_store_kernel",
                                           algorithmic_bytes_per_launch=qk_bytes, avg_launch_us=round(t_qk, 2),
                                           tokens=tokens),
        "roofline_lm_head_argmax": hbm(lm_bytes, t_lm, traffic=traffic_of("lm_head"), kernel="lm_head_argmax_kernel",
                                       algorithmic_bytes_per_launch=lm_bytes, avg_launch_us=round(t_lm, 2),
                                       rows=sample_rows, vocab=vocab, hidden=hidden,
                                       torch_linear_argmax_us=round(t_lm_torch, 2)),
        "cpu_baseline": cpu,
        # traffic and mfma_busy values above are read from these committed
        # rocprofv3 summaries, not measured in this run
        "profile_fields_from": {
            "traffic": profile_stamp(traffic, "traffic_mixed_24decode_2x512chunk.json"),
            "mfma_busy": profile_stamp(all_counters, "counters_paged_attention.json"),
        },
    }
    print(json.dumps(line))


def profile(args, device):
    """Eager launches of one kernel kind, for rocprofv3 counter and trace runs."""
    import torch
    from slo_attn import _lib, lm_head_argmax, qk_norm_rope_store, rope_cos_sin
    w = workloads.config(args.config)
    st = Step(w, device, fp8=args.kv == "fp8")
    src = torch.empty(256 << 20, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    dst.copy_(src)  # calibration: 256 MiB read + 256 MiB written
    if args.profile in ("fused", "decode", "prefill"):
        phases = {"fused": _lib.PHASE_ALL, "decode": _lib.PHASE_DECODE, "prefill": _lib.PHASE_PREFILL}[args.profile]
        fold = args.profile == "fused" and not st.fp8 and w.num_decode > 0 and bool(w.prefill_q)
        launch = lambda i: st.attn(i, phases, fold)  # noqa: E731
    elif args.profile == "qk":
        g = torch.Generator().manual_seed(5)
        qkv = torch.randn(w.num_tokens, (st.hq + 2 * st.hkv) * st.d, generator=g).to(torch.bfloat16).to(device)
        pos = torch.zeros(w.num_tokens, dtype=torch.int64, device=device)
        ones = torch.ones(st.d, dtype=torch.bfloat16, device=device)
        cs = rope_cos_sin(st.d, 4096, 1e6, device)

        def launch(i):
            kc, vc, ks, vs = st.pools[i % st.nsets]
            qk_norm_rope_store(qkv, pos, ones, ones, 1e-6, cs, st.hq, st.hkv, kc, vc, st.slots, ks, vs)
    else:
        heads = [torch.empty(151936, 2560, dtype=torch.bfloat16, device=device).normal_(0, 0.02) for _ in range(2)]
        hid = torch.randn(w.num_decode + len(w.prefill_q), 2560, dtype=torch.bfloat16, device=device)
        launch = lambda i: lm_head_argmax(hid, heads[i % 2])  # noqa: E731
    for i in range(args.events):
        launch(i)
    torch.cuda.synchronize()
    print(json.dumps({"profile": args.profile, "config": args.config, "kv": args.kv, "launches": args.events}))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for ln in fh:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def config_table(args, device):
    """Every workload config: graph-replayed step (forward_mixed, KV write included), decode-only
    and prefill-only launches on bf16 and E4M3FN pools, with the algorithmic rates, and the CPU
    oracle's time for the same step (bf16 pool) unless --no-cpu-baseline."""
    import torch
    from slo_attn import _lib
    for idx in range(5):
        w = workloads.config(idx)
        line = {"config": idx, "workload": w.name, "new_tokens": w.num_tokens, "decode_rows": w.num_decode,
                "decode_context_sum": sum(w.decode_lens), "prefill_chunks": list(w.prefill_q),
                "prefill_prefixes": list(w.prefill_prefix), "prefill_gflop": round(w.prefill_flops() / 1e9, 3)}
        for fp8 in (False, True):
            st = Step(w, device, fp8=fp8)
            r = {}
            t, _ = st.time(st.step)
            r["step_us"] = round(t, 2)
            r["step_tokens_per_s"] = round(w.num_tokens / (t * 1e-6), 1)
            if w.num_decode:
                t, _ = st.time(lambda i: st.attn(i, _lib.PHASE_DECODE))
                r["decode_us"] = round(t, 2)
                r["decode_kv_bytes"] = st.decode_bytes()
                r["decode_GBps"] = round(st.decode_bytes() / (t * 1e-6) / 1e9, 1)
                r["decode_frac_hbm"] = round(st.decode_bytes() / (t * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
            if w.prefill_q:
                t, _ = st.time(lambda i: st.attn(i, _lib.PHASE_PREFILL))
                r["prefill_us"] = round(t, 2)
                r["prefill_TFLOPs"] = round(w.prefill_flops() / (t * 1e-6) / 1e12, 1)
                r["prefill_frac_mfma"] = round(w.prefill_flops() / (t * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)
            if w.num_decode and w.prefill_q:
                r["split_us"] = round(r["decode_us"] + r["prefill_us"], 2)
            line["e4m3fn" if fp8 else "bf16"] = r
            del st
            torch.cuda.empty_cache()
        if not args.no_cpu_baseline:
            line["cpu_oracle"] = cpu_baseline(w, runs=3)
        print(json.dumps(line), flush=True)


def cpu_baseline(w, runs=5):
    """The CPU oracle (fp32 torch on the host cores) on the same step: store, then attention."""
    import torch
    from oracle import attention as oatt
    from oracle import kvstore
    from workloads import padded_tables

    meta = {
        "num_decode": w.num_decode, "num_prefill_tokens": sum(w.prefill_q), "decode_lens": w.decode_lens,
        "decode_tables": padded_tables(w.decode_tables) if w.decode_tables else [], "prefill_cu_q": w.cu_q,
        "prefill_cu_k": w.cu_k, "prefill_tables": padded_tables(w.prefill_tables) if w.prefill_tables else [],
        "prefill_has_history": w.has_history,
    }
    torch.set_num_threads(os.cpu_count() or 1)
    kc = w.k_cache.clone()
    vc = w.v_cache.clone()

    def run():
        kvstore.store_kvcache(w.k.view(torch.int16).numpy(), w.v.view(torch.int16).numpy(),
                              kc.view(torch.int16).numpy(), vc.view(torch.int16).numpy(), w.slot_mapping)
        return oatt.mixed(w.q.float(), w.k.float(), w.v.float(), kc, vc, meta, w.scale)

    run()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(w.num_tokens / t, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "cpu": cpu_model(), "kind": "port", "ms_per_step": round(t * 1e3, 1),
            "sample": f"full step ({w.num_tokens} tokens, bf16 pool): median of {runs} after 1 warm-up, "
                      f"{t * 1e3:.1f} ms per step"}


if __name__ == "__main__":
    main()
