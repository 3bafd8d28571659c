"""Benchmark of the warm partial-recompute prefill hot path on one MI355X.

Workload (N=1): Qwen2.5-VL-3B shapes (36 layers, 16 q / 2 kv heads, head_dim
128), one warm request of 128 text + 10549 image (4K, 77x137 merged grid) + 64
text tokens, recompute ratio 0.1 (1055 image tokens recomputed, 9494 reused),
image KV cached at text prefix 40 and re-rotated to prefix 128, paged KV in
256-token blocks.  Synthetic seeded N(0, 1) bf16 inputs, resident on the GPU
before the timed region.

A step = the all-layer K-rerotate + V copy of the reused image KV, then for each
of the 36 layers the fused M-RoPE of the 1247 recomputed tokens' q and k with
the store of their k and v into the paged cache, and the varlen paged GQA
causal attention of those tokens against the 10741-token cache.

value = attention microseconds per layer: the step's 36 attention calls (main
kernel + split-KV combine each, with the launch gap between them) captured as
one HIP graph and replayed once per timed step, HIP events around each replay,
divided by 36.  That is the GPU's time; HIP events around each eager call
(also reported) add the host's Python and launch time whenever the host falls
behind the GPU.  The fused RoPE + store, the separate scatter and torch's eager
RoPE (the unfused sequence the fused kernel replaces) are timed the same way.  The rerotate is
timed cold as well (a 512 MiB read before each of 10 runs leaves the MALL
holding clean lines of other data; median), next to a plain device copy of the
same bytes timed the same way; both are also reported after a 512 MiB write,
which leaves the MALL full of dirty lines whose write-backs compete.
The paged decode attention of the batched 7B tail (batch 4, ~13.4k context) is
timed cold on its own (kernels.decode); the vision tower on one 4K image (the
cold path that fills the encoder cache) is timed whole and per attention kernel.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16
HBM_PEAK_GBPS = 8000.0           # MI355X HBM3E

METRIC = "warm-prefill attn µs/layer + %MFMA peak; rerotate/scatter GB/s; warm TTFT"


def _cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def _profiled_attention_traffic(wl_name: str):
    """HBM bytes per attention call (fwd + combine) from the committed rocprofv3 PMC summary."""
    if wl_name != "cfg2":
        return None
    path = os.path.join(ROOT, "profiles", "warm_prefill_3b_4k_r0.1_hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("attention_traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _events(n):
    return [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]


def _gpu_busy():
    """A ~0.5 ms spin on the stream (no memory traffic, so the cache state a flush left
    stays): while it runs the host submits the start event, the call and the end
    event, so the events bracket the call's GPU time and not the host's submission."""
    torch.cuda._sleep(1_000_000)


def _mean_ms(evs):
    return sum(s.elapsed_time(e) for s, e in evs) / max(1, len(evs))


def _graph_us_per_call(fn_layer, num_layers: int, steps: int):
    """GPU time of one call of fn_layer(layer), averaged over the layers: the
    num_layers calls (repeated until the graph holds at least 36, so that the
    replay's own launch latency is spread over as many calls as a 36-layer step
    has) are captured in one HIP graph, replayed `steps` times with events around
    each replay.  Host time (the Python wrappers, event records) is not in the
    figure; the launch gaps between the kernels are.  None if the calls cannot be
    captured."""
    reps = max(1, -(-36 // num_layers))
    try:
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            for layer in range(num_layers):
                fn_layer(layer)
        torch.cuda.current_stream().wait_stream(st)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                for layer in range(num_layers):
                    fn_layer(layer)
        g.replay()
        torch.cuda.synchronize()
        ev = _events(steps)
        for a, b in ev:
            a.record()
            g.replay()
            b.record()
        torch.cuda.synchronize()
        return _mean_ms(ev) * 1e3 / (num_layers * reps)
    except Exception as e:  # report, do not hide
        print(f"graph timing unavailable: {e!r}", file=sys.stderr)
        return None


def _timing_note(r, name: str) -> str:
    if r["graph_timed"][name]:
        return "GPU time per call: the step's per-layer calls as one HIP graph, replayed once per timed step"
    return "HIP events around each eager call (graph capture unavailable)"


def run_gpu(steps: int, warmup: int, wl_name: str = "cfg2"):
    from vlcache_amd import workloads
    from vlcache_amd.hotpath import WarmPrefillHotPath

    wl = getattr(workloads, wl_name)()
    hp = WarmPrefillHotPath(wl, "cuda:0", seed=0)
    m = wl.model
    L = m.num_layers
    for _ in range(warmup):
        hp.step()
    torch.cuda.synchronize()

    ev_rr = _events(steps)
    ev_rs = _events(steps * L)
    ev_at = _events(steps * L)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        if hp.n_reused:
            ev_rr[s][0].record()
            hp.rerotate()
            ev_rr[s][1].record()
        for layer in range(L):
            i = s * L + layer
            ev_rs[i][0].record()
            hp.rope_store(layer)
            ev_rs[i][1].record()
            ev_at[i][0].record()
            hp.attention(layer)
            ev_at[i][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    # The same step replayed as one HIP graph (no host launch overhead).
    graph_ms = None
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            hp.step()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            hp.step()
        g.replay()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        graph_ms = (time.perf_counter() - t1) * 1e3 / steps
    except Exception as e:  # report, do not hide
        print(f"graph replay unavailable: {e!r}", file=sys.stderr)

    # The unfused sequence the fused kernel replaces, timed the same way (warm):
    # the reference's separate store_kvcache scatter, and torch's eager RoPE of q and k.
    ev_sc = _events(steps * L)
    ev_tr = _events(steps * L)
    for s in range(steps):
        for layer in range(L):
            i = s * L + layer
            ev_sc[i][0].record()
            hp.scatter(layer)
            ev_sc[i][1].record()
            ev_tr[i][0].record()
            hp.torch_rope()
            ev_tr[i][1].record()
    torch.cuda.synchronize()

    # Per-call GPU times without host time: each kernel's 36 per-layer calls as a graph.
    at_graph_us = _graph_us_per_call(hp.attention, L, steps)
    rs_graph_us = _graph_us_per_call(hp.rope_store, L, steps)
    sc_graph_us = _graph_us_per_call(hp.scatter, L, steps)
    tr_graph_us = _graph_us_per_call(lambda layer: hp.torch_rope(), L, steps)

    cu_q, cu_k = hp.cu_q_host, hp.cu_k_host
    flops = workloads.attention_flops(cu_q, cu_k, m.num_heads, m.head_dim)
    at_eager_ms = _mean_ms(ev_at)
    at_ms = at_graph_us * 1e-3 if at_graph_us else at_eager_ms
    rs_eager_ms, sc_eager_ms, tr_eager_ms = _mean_ms(ev_rs), _mean_ms(ev_sc), _mean_ms(ev_tr)
    rs_ms = rs_graph_us * 1e-3 if rs_graph_us else rs_eager_ms
    sc_ms = sc_graph_us * 1e-3 if sc_graph_us else sc_eager_ms
    tr_ms = tr_graph_us * 1e-3 if tr_graph_us else tr_eager_ms
    rr_ms = _mean_ms(ev_rr) if hp.n_reused else None
    rr_in_step_ms = rr_ms
    copy_ms = rr_dirty_ms = copy_dirty_ms = None
    if hp.n_reused:
        # Bandwidth kernels are timed cold: a 512 MiB read evicts the 256 MB MALL
        # before each run (median of 10), leaving it clean; a 512 MiB write instead
        # leaves it dirty, and that variant is reported too.  A plain device copy
        # of the same bytes, timed the same way, gives this box's copy rate.
        flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        nbytes = workloads.rerotate_bytes(hp.n_reused, L, m.num_kv_heads, m.head_dim, with_v=True) // 2
        src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)

        def cold_ms(fn, reps=10, dirty=False):
            ts = []
            for _ in range(reps):
                if dirty:
                    flush.fill_(1)
                else:
                    flush.view(torch.int64).sum()
                _gpu_busy()
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                fn()
                b.record()
                torch.cuda.synchronize()
                ts.append(a.elapsed_time(b))
            ts.sort()
            return ts[len(ts) // 2]

        rr_ms = cold_ms(hp.rerotate)
        copy_ms = cold_ms(lambda: dst.copy_(src))
        rr_dirty_ms = cold_ms(hp.rerotate, dirty=True)
        copy_dirty_ms = cold_ms(lambda: dst.copy_(src), dirty=True)
        del flush, src, dst
    at_tflops = flops / (at_ms * 1e-3) / 1e12
    sc_bytes = workloads.scatter_bytes(hp.n_computed, m.num_kv_heads, m.head_dim)
    sc_gbps = sc_bytes / (sc_ms * 1e-3) / 1e9
    rs_bytes = workloads.rope_store_bytes(hp.n_computed, m.num_heads, m.num_kv_heads, m.head_dim)
    rs_gbps = rs_bytes / (rs_ms * 1e-3) / 1e9
    rr_bytes = workloads.rerotate_bytes(hp.n_reused, L, m.num_kv_heads, m.head_dim, with_v=True)
    rr_gbps = rr_bytes / (rr_ms * 1e-3) / 1e9 if rr_ms else None
    return dict(
        wl=wl, hp=hp, wall=wall, graph_ms=graph_ms, flops=flops,
        at_us=at_ms * 1e3, at_tflops=at_tflops, sc_us=sc_ms * 1e3, sc_gbps=sc_gbps, sc_bytes=sc_bytes,
        rs_us=rs_ms * 1e3, rs_gbps=rs_gbps, rs_bytes=rs_bytes, torch_rope_us=tr_ms * 1e3,
        graph_timed={"attention": at_graph_us is not None, "rope_store": rs_graph_us is not None,
                     "scatter": sc_graph_us is not None, "torch_rope": tr_graph_us is not None},
        eager_us={"attention": at_eager_ms * 1e3, "rope_store": rs_eager_ms * 1e3,
                  "scatter": sc_eager_ms * 1e3, "torch_rope": tr_eager_ms * 1e3},
        rr_us=rr_ms * 1e3 if rr_ms else None, rr_gbps=rr_gbps, rr_bytes=rr_bytes,
        rr_in_step_us=rr_in_step_ms * 1e3 if rr_in_step_ms else None,
        copy_gbps=rr_bytes / (copy_ms * 1e-3) / 1e9 if copy_ms else None,
        rr_dirty_us=rr_dirty_ms * 1e3 if rr_dirty_ms else None,
        copy_dirty_gbps=rr_bytes / (copy_dirty_ms * 1e-3) / 1e9 if copy_dirty_ms else None,
        plan=(hp.plan.num_items, hp.plan.num_combine),
    )


def _cold_ms(fn, flush, reps=5, dirty=False):
    """Median GPU time of fn() after a 512 MiB read (MALL left holding clean lines) or
    write (dirty lines), with the events behind a GPU spin."""
    ts = []
    for _ in range(reps):
        if dirty:
            flush.fill_(1)
        else:
            flush.view(torch.int64).sum()
        _gpu_busy()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b))
    ts.sort()
    return ts[len(ts) // 2]


def run_config(wl_name: str, steps: int, warmup: int, scatter: bool = False):
    """The other workloads' kernels, each timed as in the main line: attention and the
    fused RoPE + store as the step's per-layer calls in one HIP graph (per call), the
    re-rotation cold (median of 5)."""
    from vlcache_amd import workloads
    from vlcache_amd.hotpath import WarmPrefillHotPath

    wl = getattr(workloads, wl_name)()
    hp = WarmPrefillHotPath(wl, "cuda:0", seed=0)
    m = wl.model
    L = m.num_layers
    for _ in range(warmup):
        hp.step()
    torch.cuda.synchronize()
    reps = max(2, min(steps, 5))
    at_us = _graph_us_per_call(hp.attention, L, reps)
    rs_us = _graph_us_per_call(hp.rope_store, L, reps)
    flops = workloads.attention_flops(hp.cu_q_host, hp.cu_k_host, m.num_heads, m.head_dim)
    tflops = flops / (at_us * 1e-6) / 1e12
    rs_bytes = workloads.rope_store_bytes(hp.n_computed, m.num_heads, m.num_kv_heads, m.head_dim)
    out = {
        "workload": f"{wl.name}: {m.name}, {L} layers, heads {m.num_heads}/{m.num_kv_heads}, "
                    f"{len(wl.requests)} request(s), {hp.n_computed} computed / {hp.n_reused} reused tokens, "
                    f"{len(hp.cu_q_host) - 1} virtual sub-sequences",
        "attention": {"us_per_layer": round(at_us, 2), "gflop_per_layer": round(flops / 1e9, 3),
                      "tflops": round(tflops, 1), "frac_mfma_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                      "work_items": hp.plan.num_items, "split_combines": hp.plan.num_combine,
                      "paged": hp.paged},
        "rope_store": {"us_per_layer": round(rs_us, 2), "bytes": rs_bytes,
                       "gbps": round(rs_bytes / (rs_us * 1e-6) / 1e9, 1),
                       "frac_hbm_peak": round(rs_bytes / (rs_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)},
        "timing": "per call: the step's per-layer calls captured as one HIP graph, replayed, HIP events",
    }
    if scatter:
        sc_us = _graph_us_per_call(hp.scatter, L, reps)
        sc_bytes = workloads.scatter_bytes(hp.n_computed, m.num_kv_heads, m.head_dim)
        out["scatter"] = {"us_per_layer": round(sc_us, 2), "bytes": sc_bytes,
                          "gbps": round(sc_bytes / (sc_us * 1e-6) / 1e9, 1),
                          "frac_hbm_peak": round(sc_bytes / (sc_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
    if hp.n_reused:
        flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        rr_bytes = workloads.rerotate_bytes(hp.n_reused, L, m.num_kv_heads, m.head_dim, with_v=True)
        rr_ms = _cold_ms(hp.rerotate, flush)
        rr_dirty_ms = _cold_ms(hp.rerotate, flush, dirty=True)
        out["rerotate"] = {"us_all_layers": round(rr_ms * 1e3, 1), "bytes": rr_bytes,
                           "gbps": round(rr_bytes / (rr_ms * 1e-3) / 1e9, 1),
                           "frac_hbm_peak": round(rr_bytes / (rr_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                           "dirty_mall_us": round(rr_dirty_ms * 1e3, 1),
                           "timing": "cold: 512 MiB read (clean MALL) or write (dirty) before each run, median of 5"}
        del flush
    del hp
    torch.cuda.empty_cache()
    return out


SWEEP_TOKENS = (256, 1247, 4096, 10741, 32768)


def run_bandwidth_sweep(tokens=SWEEP_TOKENS, steps: int = 5):
    """The two per-layer bandwidth kernels over a range of recomputed-token counts, on
    Qwen2.5-VL-3B shapes (16/2 heads, head_dim 128, pages of 256), next to a plain
    device copy that reads and writes the scatter's bytes: where the kernels and the
    copy both fall short of the large-size rate, the size is launch-bound, not the
    kernel.  Each figure is per call, 36 calls (one per layer, distinct caches) in one
    HIP graph, as in the main line."""
    from vlcache_amd import kernels
    from vlcache_amd.hotpath import MAX_POSITIONS
    from vlcache_amd.layers.rotary_embedding import get_rope
    from vlcache_amd.workloads import BLOCK_SIZE, QWEN25_VL_3B as m, rope_store_bytes, scatter_bytes

    dev = torch.device("cuda:0")
    hq, hkv, hd, L = m.num_heads, m.num_kv_heads, m.head_dim, m.num_layers
    rope = get_rope(hd, hd, MAX_POSITIONS, m.rope_theta, {"mrope_section": list(m.mrope_section)}).to(dev)
    out = {"tokens": list(tokens), "scatter_us": [], "scatter_gbps": [], "rope_store_us": [],
           "rope_store_gbps": [], "copy_us": [], "copy_gbps": [],
           "copy": "torch copy_ reading and writing the scatter's bytes (K and V rows)",
           "timing": "per call: 36 calls (distinct per-layer caches) in one HIP graph, replayed, HIP events"}
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    for n in tokens:
        nb = -(-n // BLOCK_SIZE)
        qkv = torch.randn(n, (hq + 2 * hkv) * hd, generator=g, device=dev, dtype=torch.bfloat16)
        q_in = qkv[:, :hq * hd].view(n, hq, hd)
        k_in = qkv[:, hq * hd:(hq + hkv) * hd].view(n, hkv, hd)
        v = qkv[:, (hq + hkv) * hd:].view(n, hkv, hd)
        k = k_in.contiguous()
        q = torch.empty(n, hq, hd, device=dev, dtype=torch.bfloat16)
        kc = torch.zeros(L, nb, BLOCK_SIZE, hkv, hd, device=dev, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        # the engine's layout: a sequence's tokens fill its pages in order, pages in any order
        pages = torch.randperm(nb, generator=g, device=dev)
        tok = torch.arange(n, device=dev)
        slots = (pages[tok // BLOCK_SIZE] * BLOCK_SIZE + tok % BLOCK_SIZE).to(torch.int32)
        pos = torch.randint(0, 4096, (3, n), generator=g, device=dev, dtype=torch.int64)
        src = torch.randn(n, 2 * hkv * hd, generator=g, device=dev, dtype=torch.bfloat16)
        dst = torch.empty(L, n, 2 * hkv * hd, device=dev, dtype=torch.bfloat16)
        sc = _graph_us_per_call(lambda l: kernels.store_kvcache_raw(k, v, kc[l], vc[l], slots), L, steps)
        rs = _graph_us_per_call(lambda l: kernels.rope_store_kvcache(pos, q_in, k_in, v, rope.cos_sin_cache,
                                                                     m.mrope_section, kc[l], vc[l], slots,
                                                                     q_out=q), L, steps)
        cp = _graph_us_per_call(lambda l: dst[l].copy_(src), L, steps)
        sb, rb = scatter_bytes(n, hkv, hd), rope_store_bytes(n, hq, hkv, hd)
        for key, us, b in (("scatter", sc, sb), ("rope_store", rs, rb), ("copy", cp, sb)):
            out[f"{key}_us"].append(None if us is None else round(us, 2))
            out[f"{key}_gbps"].append(None if us is None else round(b / (us * 1e-6) / 1e9, 1))
        del qkv, q, k, kc, vc, src, dst
    torch.cuda.empty_cache()
    return out


def run_ttft(ratio: float, reps: int = 2):
    """Warm TTFT (ms) of the cold -> warm protocol of the reference's test_partial_recompute.py.

    Random-init Qwen2.5-VL-3B (36 text layers, 32-block vision tower); each image
    is the 4K grid (1, 154, 274): 42196 patches of random pixels -> 10549 tokens.
    Per repetition, a fresh image is sent cold (text prefix 40, suffix 64: the
    vision tower runs and fills the encoder cache) and then warm (prefix 128,
    suffix 64: a cache hit).  TTFT is the engine's own clock: from request
    creation to the sampled first token on the host; vit_ms is the vision
    tower's share of the cold request.  The first repetition warms up kernels
    and libraries and is not reported.
    """
    import numpy as np

    from vlcache_amd import LLM, SamplingParams
    from vlcache_amd.config import QWEN25_VL_3B

    img_tok = QWEN25_VL_3B["image_token_id"]
    llm = LLM(dict(QWEN25_VL_3B), recompute_ratio=ratio, num_kvcache_blocks=8 * 43, enforce_eager=True)
    sp = SamplingParams(temperature=0.6, max_tokens=1)
    grid = torch.tensor([[1, 154, 274]])
    n_img = 77 * 137
    rng = np.random.default_rng(0)

    def prompt(prefix, suffix):
        return ([int(x) for x in rng.integers(1, 150000, prefix)] + [img_tok] * n_img
                + [int(x) for x in rng.integers(1, 150000, suffix)])

    cold, warm, vit = [], [], []
    for r in range(reps + 1):
        # a distinct image per repetition: processor-shaped patches [42196, 3*2*14*14] fp32
        pv = torch.randn(154 * 274, 1176, generator=torch.Generator().manual_seed(100 + r))
        mm = {"pixel_values": pv, "image_grid_thw": grid}
        o1 = llm.generate([prompt(40, 64)], sp, mm_inputs=[mm])
        o2 = llm.generate([prompt(128, 64)], sp, mm_inputs=[mm])
        assert o1[0]["vit_time"] > 0 and o2[0]["vit_time"] == 0.0
        if r > 0:
            cold.append(o1[0]["ttft"] * 1e3)
            warm.append(o2[0]["ttft"] * 1e3)
            vit.append(o1[0]["vit_time"] * 1e3)
    del llm
    torch.cuda.empty_cache()
    return {"cold_ms": round(float(np.median(cold)), 2), "warm_ms": round(float(np.median(warm)), 2),
            "vit_ms": round(float(np.median(vit)), 2)}


def run_decode(reps: int = 10):
    """Paged GQA decode attention of the batched 7B request tail: batch 4 at contexts
    13432..13435 tokens, 28 q / 4 kv heads, 256-token pages in a seeded permutation.

    Each layer of a decode step reads a different layer's cache (28 x 110 MB), so
    every read is cold: a 512 MiB read before each timed call leaves the MALL full
    of clean lines (median of `reps`).  The same bytes are timed through the
    varlen prefill kernel (one query per sequence) for comparison.
    """
    from vlcache_amd import kernels

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    B, hq, hkv, page = 4, 28, 4, 256
    lens = [13432 + i for i in range(B)]
    nbs = [-(-n // page) for n in lens]
    nb = sum(nbs)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(7)).to(torch.int32)
    bt = torch.full((B, max(nbs)), -1, dtype=torch.int32)
    p0 = 0
    for i, n in enumerate(nbs):
        bt[i, :n] = perm[p0:p0 + n]
        p0 += n
    bt = bt.to(dev)
    q = torch.randn(B, hq, 128, generator=g, device=dev, dtype=torch.bfloat16)
    kc = torch.randn(nb, page, hkv, 128, generator=g, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(nb, page, hkv, 128, generator=g, device=dev, dtype=torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    plan = kernels.plan_decode(B, hq, hkv, 128, page, max(lens), dev)
    out = torch.empty(B, hq, 128, dtype=torch.bfloat16, device=dev)
    cu_q = list(range(B + 1))
    cu_k = [0]
    for n in lens:
        cu_k.append(cu_k[-1] + n)
    vplan = kernels.plan_attention(cu_q, cu_k, hq, hkv, 128, True, dev)
    cq = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    ck = torch.tensor(cu_k, dtype=torch.int32, device=dev)
    out2 = torch.empty_like(out)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)

    def timed(fn, cold):
        for _ in range(2):
            fn()
        ts = []
        for _ in range(reps):
            if cold:
                flush.view(torch.int64).sum()  # read-only: the MALL ends up holding clean lines
            _gpu_busy()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b) * 1e3)
        ts.sort()
        return ts[len(ts) // 2]

    dec = lambda: kernels.decode_attention(q, kc, vc, sl, bt, 128 ** -0.5, plan=plan, out=out)
    var = lambda: kernels.varlen_attention(q, kc, vc, cq, ck, 128 ** -0.5, True, bt, plan=vplan, out=out2)
    nbytes = sum(lens) * hkv * 128 * 2 * 2
    res = {"cold_us": timed(dec, True), "varlen_path_cold_us": timed(var, True)}
    del flush
    torch.cuda.synchronize()
    err = (out.float() - out2.float()).abs().max().item()
    del kc, vc
    # As in a decode step: 28 layers' caches (3.1 GB, far beyond the 256 MB MALL, so every
    # call reads cold lines), one call per layer, captured as one HIP graph.
    L = 28
    kc_all = torch.randn(L, nb, page, hkv, 128, generator=g, device=dev, dtype=torch.bfloat16)
    vc_all = torch.randn(L, nb, page, hkv, 128, generator=g, device=dev, dtype=torch.bfloat16)
    step_us = _graph_us_per_call(
        lambda l: kernels.decode_attention(q, kc_all[l], vc_all[l], sl, bt, 128 ** -0.5, plan=plan, out=out), L, 5)
    del kc_all, vc_all
    torch.cuda.empty_cache()
    cold_gbps = nbytes / (res["cold_us"] * 1e-6) / 1e9
    us = step_us if step_us is not None else res["cold_us"]
    gbps = nbytes / (us * 1e-6) / 1e9
    return {
        "workload": "batch 4 decode, contexts 13432..13435, 28/4 heads x 128, pages of 256",
        "bytes": nbytes, "us_per_layer": round(us, 2), "gbps": round(gbps, 1),
        "frac_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "timing": ("as in a decode step: 28 calls, one per layer's cache (3.1 GB in all, far beyond the "
                   "256 MB MALL, so every call reads cold lines), in one HIP graph, replayed, per call"
                   if step_us is not None else "cold single call (graph capture unavailable)"),
        "cold_single_call": {
            "us": round(res["cold_us"], 2), "gbps": round(cold_gbps, 1),
            "timing": ("512 MiB read before each call (MALL holds clean lines), median of 10; events "
                       "bracket the call behind a GPU spin, so host submission is excluded but the event "
                       "pair's own few us are not")},
        "varlen_path_cold_us": round(res["varlen_path_cold_us"], 2),
        "key_chunk": plan.key_chunk, "chunks": plan.grid_splits, "pipeline": hex(plan.pipeline),
        "max_abs_vs_varlen_path": err,
    }


def run_decode_tail(steps: int = 128):
    """The two-image 7B batch through the engine, then its decode tail.

    Random-init Qwen2.5-VL-7B (28 text layers, 32-block vision tower).  Two cold
    requests (64 text + image + 64 text, for a 1920x1080 and a 4K image of random
    pixels) fill the encoder and image-KV caches; then 4 warm requests of 64 text +
    1080p image + 64 text + 4K image + 64 text = 13432 tokens (ratio 0.02: 54 + 211
    image tokens recomputed) generate `steps` tokens each (ignore_eos), once with
    the decode steps replaying captured HIP graphs (enforce_eager=False, the
    reference's default) and once eagerly.  A warm-up batch of 8 tokens comes first
    (it captures the batch-4 graph).  decode_ms_per_step = (wall time of the
    generate call - the latest first token's TTFT) / (steps - 1): every step after
    the prefill is a decode step of the batch of 4 at 13.4k-13.6k context.
    """
    import numpy as np

    from vlcache_amd import LLM, SamplingParams
    from vlcache_amd.config import QWEN25_VL_7B

    img = QWEN25_VL_7B["image_token_id"]
    llm = LLM(dict(QWEN25_VL_7B), recompute_ratio=0.02, num_kvcache_blocks=640, enforce_eager=False,
              max_model_len=16384, max_num_batched_tokens=32768, max_num_seqs=16)
    runner = llm.model_runner
    rng = np.random.default_rng(5)
    g1, g2 = (1, 78, 138), (1, 154, 274)          # 39 x 69 = 2691 and 77 x 137 = 10549 tokens
    n1, n2 = 39 * 69, 77 * 137
    gen = torch.Generator().manual_seed(11)
    p1 = torch.randn(g1[1] * g1[2], 1176, generator=gen)
    p2 = torch.randn(g2[1] * g2[2], 1176, generator=gen)

    def text(n):
        return [int(x) for x in rng.integers(1, 150000, n)]

    cold = [text(64) + [img] * n1 + text(64), text(64) + [img] * n2 + text(64)]
    cold_mm = [{"pixel_values": p1, "image_grid_thw": torch.tensor([list(g1)])},
               {"pixel_values": p2, "image_grid_thw": torch.tensor([list(g2)])}]
    llm.generate(cold, SamplingParams(temperature=0.6, max_tokens=1), mm_inputs=cold_mm)
    warm_mm = {"pixel_values": torch.cat([p1, p2]), "image_grid_thw": torch.tensor([list(g1), list(g2)])}

    def batch():
        return [text(64) + [img] * n1 + text(64) + [img] * n2 + text(64) for _ in range(4)]

    llm.generate(batch(), SamplingParams(temperature=0.6, max_tokens=8, ignore_eos=True), mm_inputs=[warm_mm] * 4)
    out = {"workload": "Qwen2.5-VL-7B (random init), batch 4 x (64 + 2691 + 64 + 10549 + 64) tokens, ratio 0.02, "
                       f"both images cached; {steps} tokens per request"}
    for mode, eager in (("graphs", False), ("eager", True)):
        runner.enforce_eager = eager
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        outs = llm.generate(batch(), SamplingParams(temperature=0.6, max_tokens=steps, ignore_eos=True),
                            mm_inputs=[warm_mm] * 4)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ttft = max(o["ttft"] for o in outs)
        assert all(len(o["token_ids"]) == steps for o in outs)
        assert all(o["vit_time"] == 0.0 for o in outs), "warm requests must hit the encoder cache"
        step_ms = (wall - ttft) * 1e3 / (steps - 1)
        out[mode] = {"warm_batch_ttft_ms": round(ttft * 1e3, 2), "decode_ms_per_step": round(step_ms, 3),
                     "decode_tokens_per_s": round(4 * 1e3 / step_ms, 1)}
    out["timing"] = ("engine wall clock after a cold pass and a warm-up batch; 'graphs': decode steps replay "
                     "captured HIP graphs, 'eager': the same engine with graph replay off")
    del llm, runner
    torch.cuda.empty_cache()
    return out


def run_vision(reps: int = 5):
    """The vision tower on one 4K image (grid (1, 154, 274): 42196 patches -> 10549 tokens).

    Random-init public configuration (32 blocks of hidden 1280, 16 heads of 80 dims,
    whole-image attention at blocks 7/15/23/31, window 112 px).  Whole forward:
    HIP events around each of `reps` calls after one warm-up, median.  The three
    kernels of a block's attention on the same layout, each the median of 20
    event-timed calls: the fused rotary + head padding (HBM: bytes read + written),
    the window attention and the whole-image attention (MFMA: 4 * pairs * 80 dims
    * 16 heads; the kernel's 80-dim variant skips the heads' zero padding; HBM: the q, k, v
    head rows read once and the output written once, which bounds the window attention's
    64-token windows).
    """
    from vlcache_amd import kernels
    from vlcache_amd.config import QWEN25_VL_VISION
    from vlcache_amd.qwen_vl import random_init_
    from vlcache_amd.vision import VisionTransformer, vision_config

    dev = torch.device("cuda:0")
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            vt = VisionTransformer(vision_config(dict(QWEN25_VL_VISION), 2048))
    finally:
        torch.set_default_dtype(prev)
    random_init_(vt)
    vt.eval()
    grids = [(1, 154, 274)]
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    pix = torch.randn(154 * 274, 1176, generator=g, device=dev)
    vt(pix, grids)
    torch.cuda.synchronize()
    ev = _events(reps)
    for a, b in ev:
        a.record()
        vt(pix, grids)
        b.record()
    torch.cuda.synchronize()
    fwd = sorted(a.elapsed_time(b) for a, b in ev)[reps // 2]
    run = vt._prepare(grids)
    lay = run.layout
    n, h, hd = lay.num_patches, vt.cfg.num_heads, vt.head_dim
    qkv = torch.randn(n, 3 * h * hd, generator=g, device=dev, dtype=torch.bfloat16)
    heads = kernels.vision_rope_pad(qkv, run.pos_hw, run.cos, run.sin, h, hd)
    o = torch.empty(n, h, kernels.HEAD_DIM, dtype=torch.bfloat16, device=dev)

    def med_ms(fn, k=20):
        fn()
        torch.cuda.synchronize()
        e = _events(k)
        for a, b in e:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        return sorted(a.elapsed_time(b) for a, b in e)[k // 2]

    rope_ms = med_ms(lambda: kernels.vision_rope_pad(qkv, run.pos_hw, run.cos, run.sin, h, hd, out=heads))
    rope_bytes = n * (3 * h * hd * 2 + 3 * h * kernels.HEAD_DIM * 2)

    def attn(cu, plan):
        return lambda: kernels.varlen_attention(heads[:, 0], heads[:, 1], heads[:, 2], cu, cu, hd ** -0.5,
                                                causal=False, plan=plan, out=o, head_dim=run.attn_head_dim)

    out = {"workload": "Qwen2.5-VL vision tower (public config, random init), one 4K image: grid (1, 154, 274), "
                       "42196 patches -> 10549 tokens",
           "forward_ms": round(fwd, 2), "timing": f"HIP events, median of {reps} forwards after 1 warm-up",
           "rope_pad": {"ms": round(rope_ms, 4), "bytes": rope_bytes,
                        "gbps": round(rope_bytes / (rope_ms * 1e-3) / 1e9, 1),
                        "frac_hbm_peak": round(rope_bytes / (rope_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}}
    for name, cu_host, cu, plan in (("window_attention", lay.cu_window, run.cu_window, run.plan_window),
                                    ("whole_image_attention", lay.cu_full, run.cu_full, run.plan_full)):
        ms = med_ms(attn(cu, plan))
        pairs = sum((b - a) ** 2 for a, b in zip(cu_host, cu_host[1:]))
        tf = 4.0 * pairs * hd * h / (ms * 1e-3) / 1e12
        # bytes the kernel moves at least: q, k and v head rows read (128-element rows), output written
        nbytes = 4 * n * h * kernels.HEAD_DIM * 2
        out[name] = {"ms": round(ms, 4), "sequences": len(cu_host) - 1, "work_items": plan.num_items,
                     "kernel_head_dim": run.attn_head_dim, "tflops": round(tf, 1),
                     "frac_mfma_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                     "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    del vt, heads, o, qkv
    torch.cuda.empty_cache()
    return out


def _cpu_median(fn, runs: int, budget_s: float):
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s or len(times) >= runs:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def run_cpu_baseline(hp, budget_s: float = 12.0):
    """The oracle (fp32 torch on the host CPU) on bounded samples of the same workload:
    one layer's attention, the all-layer re-rotation + copy of the reused image KV, and
    one layer's store_kvcache scatter (the reference's CPU-runnable restatements)."""
    from oracle import attention as oattn
    from oracle import rope as orope
    from oracle import scatter as oscat

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    m = hp.model
    kc = hp.k_caches[0].cpu()
    vc = hp.v_caches[0].cpu()
    q = hp.q.cpu()
    bt = hp.block_tables.cpu().tolist()
    cu_q, cu_k = hp.cu_q_host, hp.cu_k_host
    at_s, at_n = _cpu_median(lambda: oattn.varlen_attention(q, kc, vc, cu_q, cu_k, hp.scale, True, bt, 256),
                             5, budget_s)
    kv = hp.kv_cache.cpu()
    old, new = hp.old_slots.cpu(), hp.new_slots.cpu()
    cs = orope.rerotation_cos_sin(hp.deltas, m.head_dim, m.rope_theta, list(m.mrope_section))
    seg = hp.seg.cpu()
    rr_s, rr_n = _cpu_median(lambda: orope.rerotate_copy_kv(kv, old, new, cs, seg), 3, budget_s)
    del kv
    k_rows = hp.k.cpu()
    v_rows = hp.v.cpu().contiguous()
    slots = hp.slot_mapping.cpu().numpy()
    kcache, vcache = kc.view(torch.int16).numpy(), vc.view(torch.int16).numpy()
    kn, vn = k_rows.view(torch.int16).numpy(), v_rows.view(torch.int16).numpy()
    sc_s, sc_n = _cpu_median(lambda: oscat.store_kvcache(kn, vn, kcache, vcache, slots), 20, budget_s / 4)
    from vlcache_amd import workloads

    rr_bytes = workloads.rerotate_bytes(hp.n_reused, m.num_layers, m.num_kv_heads, m.head_dim, with_v=True)
    sc_bytes = workloads.scatter_bytes(hp.n_computed, m.num_kv_heads, m.head_dim)
    return {
        "value": at_s * 1e6,
        "unit": "us/layer (attention)",
        "cores": cores,
        "kind": "port",
        "sample": f"{at_n} runs of one layer's attention of the same workload (fp32 SDPA oracle, median); "
                  f"re-rotation + copy: {rr_n} runs of all {m.num_layers} layers; scatter: {sc_n} runs of one "
                  f"layer; host CPU: {_cpu_model()}",
        "kernels": {
            "rerotate_copy": {"us_all_layers": round(rr_s * 1e6, 1), "gbps": round(rr_bytes / rr_s / 1e9, 2)},
            "scatter": {"us_per_layer": round(sc_s * 1e6, 1), "gbps": round(sc_bytes / sc_s / 1e9, 2)},
        },
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="cfg2")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ttft", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-vision", action="store_true", help="skip the vision tower sub-result")
    ap.add_argument("--no-decode-tail", action="store_true", help="skip the 7B batch's decode tail")
    ap.add_argument("--no-configs", action="store_true", help="skip the other workloads' sub-results")
    ap.add_argument("--no-sweep", action="store_true", help="skip the bandwidth kernels' size sweep")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only run one plain device-to-device copy of this many MiB (HBM counter calibration)")
    args = ap.parse_args()
    if args.copy_calibration_mib:
        n = args.copy_calibration_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    r = run_gpu(args.steps, args.warmup, args.workload)
    decode = run_decode() if not args.no_decode else None
    vision = run_vision() if not args.no_vision else None
    decode_tail = run_decode_tail() if not args.no_decode_tail else None
    others = {}
    if not args.no_configs:
        for name, kw in (("cfg1", {"scatter": True}), ("cfg3", {"scatter": True}), ("cfg4", {}), ("cfg5", {})):
            if name != args.workload:
                others[name] = run_config(name, args.steps, 1, **kw)
    sweep = run_bandwidth_sweep() if not args.no_sweep else None
    wl, hp = r["wl"], r["hp"]
    ttft = None
    if not args.no_ttft:
        partial = run_ttft(wl.requests[0].ratio or 0.1)
        full = run_ttft(0.0)
        ttft = {"warm_partial_ms": partial["warm_ms"], "warm_full_recompute_ms": full["warm_ms"],
                "cold_ms": partial["cold_ms"], "cold_vit_ms": partial["vit_ms"],
                "speedup_vs_full": round(full["warm_ms"] / partial["warm_ms"], 3),
                "protocol": "cold (prefix 40, vision tower runs) then warm (prefix 128, encoder-cache hit) "
                            "request, same 4K image, suffix 64, random-init 3B (36 text layers, 32 vision "
                            "blocks), median of 2 after 1 warm-up"}
    cpu = None if args.no_cpu_baseline else run_cpu_baseline(hp)
    frac = r["at_tflops"] / MFMA_BF16_PEAK_TFLOPS
    line = {
        "metric": METRIC,
        "value": round(r["at_us"], 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall"] * 1e3 / args.steps, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 q/k/v and cached KV)",
        "config": {
            "workload": f"{wl.name}: {wl.model.name} shapes, {wl.model.num_layers} layers, heads "
                        f"{wl.model.num_heads}/{wl.model.num_kv_heads}x{wl.model.head_dim}, "
                        f"{len(wl.requests)} x ("
                        + "+".join(str(v if k == 'text' else v[0] * v[1]) for k, v in wl.requests[0].parts())
                        + f") tokens, ratio {wl.requests[0].ratio}, paged blocks of 256",
            "recomputed_tokens": hp.n_computed,
            "reused_tokens": hp.n_reused,
            "cu_seqlens_q": hp.cu_q_host,
            "cu_seqlens_k": hp.cu_k_host,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(r["at_tflops"], 2),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(frac, 4),
            "traffic": _profiled_attention_traffic(args.workload),
            "traffic_source": ("not measured in this run: HBM bytes per call (attn_fwd + attn_combine) from "
                               "profiles/warm_prefill_3b_4k_r0.1_hbm_traffic.md, rocprofv3 FETCH_SIZE and "
                               "WRITE_SIZE per dispatch scaled by a plain copy's readings"
                               if args.workload == "cfg2" else "no traffic profile for this workload"),
        },
        "cpu_baseline": cpu,
        "kernels": {
            "attention": {"us_per_layer": round(r["at_us"], 3), "gflop_per_layer": round(r["flops"] / 1e9, 3),
                          "tflops": round(r["at_tflops"], 2), "frac_mfma_peak": round(frac, 4),
                          "work_items": r["plan"][0], "split_combines": r["plan"][1],
                          "timing": _timing_note(r, "attention"),
                          "eager_event_us_per_layer": round(r["eager_us"]["attention"], 3)},
            "rope_store": {"us_per_layer": round(r["rs_us"], 3), "bytes": r["rs_bytes"],
                           "gbps": round(r["rs_gbps"], 1), "frac_hbm_peak": round(r["rs_gbps"] / HBM_PEAK_GBPS, 4),
                           "replaces_us_per_layer": round(r["torch_rope_us"] + r["sc_us"], 3),
                           "replaces": "torch eager M-RoPE of q and k + store_kvcache scatter",
                           "timing": _timing_note(r, "rope_store"),
                           "eager_event_us_per_layer": round(r["eager_us"]["rope_store"], 3)},
            "scatter": {"us_per_layer": round(r["sc_us"], 3), "bytes": r["sc_bytes"],
                        "gbps": round(r["sc_gbps"], 1), "frac_hbm_peak": round(r["sc_gbps"] / HBM_PEAK_GBPS, 4),
                        "timing": "reference-API store_kvcache, outside the step; " + _timing_note(r, "scatter"),
                        "eager_event_us_per_layer": round(r["eager_us"]["scatter"], 3)},
            "torch_rope": {"us_per_layer": round(r["torch_rope_us"], 3), "timing": _timing_note(r, "torch_rope"),
                           "eager_event_us_per_layer": round(r["eager_us"]["torch_rope"], 3)},
            "decode": decode,
            "rerotate": None if r["rr_us"] is None else {
                "us_all_layers": round(r["rr_us"], 2), "bytes": r["rr_bytes"], "gbps": round(r["rr_gbps"], 1),
                "frac_hbm_peak": round(r["rr_gbps"] / HBM_PEAK_GBPS, 4),
                "timing": ("cold: 512 MiB read before each run (MALL holds clean lines), median of 10; "
                           "events bracket the call behind a GPU spin"),
                "us_in_step": round(r["rr_in_step_us"], 2),
                "plain_copy_same_bytes_gbps": round(r["copy_gbps"], 1),
                "dirty_mall": {"us_all_layers": round(r["rr_dirty_us"], 2),
                               "gbps": round(r["rr_bytes"] / (r["rr_dirty_us"] * 1e-6) / 1e9, 1),
                               "plain_copy_same_bytes_gbps": round(r["copy_dirty_gbps"], 1),
                               "timing": "512 MiB write before each run (MALL full of dirty lines)"}},
        },
        "ms_per_step_graph": None if r["graph_ms"] is None else round(r["graph_ms"], 4),
        "warm_ttft": ttft,
        "vision": vision,
        "decode_tail": decode_tail,
        "configs": others,
        "bandwidth_sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
