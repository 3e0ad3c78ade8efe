"""Benchmark of the forecast-guided block-sparse attention layer on one MI355X.

Headline (``value``): sparse prefill throughput (tok/s) of one attention
layer at B=4, T=4096, 12 query / 4 KV heads, head dim 64, block 64 (64
blocks), top-8, bf16 — one step = block compression + fused routing +
block-sparse MFMA prefill, inputs resident in HBM.

Also reported (``decode``): the decode step at a 16K context, B=8, bf16 KV
cache [8,16384,4,64], 256 blocks, top-8 + sink + current block — one step =
whole-cache compression + routing + split-K attention + combine, over >= 4
rotating cache copies (more than the 256 MB Infinity Cache), replayed from a
HIP graph.

Roofline: the prefill attention kernel against dense bf16 MFMA peak
(2.5 PFLOP/s) with useful FLOPs 4*D*sum|allowed| counted from the produced
selection lists; the decode step against HBM peak (8 TB/s) with its
algorithmic bytes. Kernel durations come from HIP events on the launch stream.

cpu_baseline: the op-for-op PyTorch restatement of the reference path
(O(T^2) masks + masked SDPA) timed on the host cores, N threads and 1
thread, warm-up 3 / runs 10, median (the reference's latency protocol).

    python bench.py [--steps K] [--warmup W] [--decode-steps N] [--no-cpu-baseline]
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "local-research-small-language-model_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "sparse-attn prefill tok/s & decode us/step @16K ctx; % HBM/MFMA roofline"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

# prefill workload
PB, PT, HQ, HKV, D, BS, TOPK = 4, 4096, 12, 4, 64, 64, 8
# decode workload
DB, DS = 8, 16384
N_CACHES = 4
# offload workload
OB_LAYERS, OB_CTX = 12, 32768
# 12-layer forward workload
MT = 16384
# plain copy used to calibrate the HBM byte counters
COPY_BYTES = 256 << 20


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--offload-steps", type=int, default=32)
    ap.add_argument("--generate-steps", type=int, default=128)
    ap.add_argument("--only", choices=["all", "prefill", "prefill16k", "decode", "offload", "model", "producer",
                                       "teacher", "generate", "pmc"],
                    default="all",
                    help="run one workload (for profiling); the JSON line needs 'all'")
    return ap.parse_args()


def events_ms(fn, reps, torch):
    """Average milliseconds of fn() over reps launches, HIP events on the current stream."""
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        fn()
    e1.record(s)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


def load_traffic():
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def bench_prefill(args, torch, sparda, synth, B=PB, T=PT, seed=1001, BS=BS, TOPK=TOPK):
    """One sparse prefill layer at [B, T] (12/4 heads, D 64, block BS, top-TOPK).
    The step: compress, then the routed prefill (the attention kernel routes its
    own windows; one launch). Beside it the two-launch form (route, then the
    prefill on the lists) for the router's own time. Eager steps with events
    around each launch, then each step replayed from a HIP graph."""
    x = synth.prefill_inputs(B, T, HQ, HKV, D, dtype=torch.bfloat16, seed=seed, device="cuda")
    q, k, v, f = x["q"], x["k"], x["v"], x["forecast"]
    out = torch.empty((B, T, HQ * D), dtype=torch.bfloat16, device="cuda")
    out2 = torch.empty_like(out)
    out3 = torch.empty_like(out) if T > 8192 else None
    state = {}

    def routed(ev=None):
        # ev: 3 events bracketing the two launches (same stream as the kernels)
        if ev is not None:
            ev[0].record()
        protos = sparda.compress(k, BS)
        if ev is not None:
            ev[1].record()
        sparda.prefill_routed(q, k, v, f, protos, BS, TOPK, out=out)
        if ev is not None:
            ev[2].record()

    def two_launch(ev=None):
        # ev: 4 events bracketing the three launches
        if ev is not None:
            ev[0].record()
        protos = sparda.compress(k, BS)
        if ev is not None:
            ev[1].record()
        _, _, sel, n = sparda.route(f, protos, BS, TOPK, want_topk=False, want_sel=True)
        if ev is not None:
            ev[2].record()
        sparda.prefill(q, k, v, sel, n, BS, out=out2)
        if ev is not None:
            ev[3].record()
        state["sel"], state["n"] = sel, n

    def chunked(ev=None):
        # the reference's path past 8192 tokens (sparse.py:284-364): every
        # row's non-causal top-k, then one launch that builds each query
        # block's list and attends over it; ev: 4 events bracketing the three
        # launches
        if ev is not None:
            ev[0].record()
        protos = sparda.compress(k, BS)
        if ev is not None:
            ev[1].record()
        topk = sparda.route(f, protos, BS, TOPK, causal=False)[0]
        if ev is not None:
            ev[2].record()
        sparda.prefill_chunked(q, k, v, topk, BS, TOPK, out=out3)
        if ev is not None:
            ev[3].record()
        state["ctopk"] = topk

    def eager(step, n_ev):
        for _ in range(args.warmup):
            step()
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(n_ev)] for _ in range(args.steps)]
        torch.cuda.synchronize()
        for ev in evs:
            step(ev)
        evs[-1][-1].synchronize()
        torch.cuda.synchronize()
        total = evs[0][0].elapsed_time(evs[-1][-1]) / args.steps
        per = [sum(e[i].elapsed_time(e[i + 1]) for e in evs) / args.steps for i in range(n_ev - 1)]
        return total, per

    def graphed(step, dst):
        # the step as a serving loop issues it: its launches recorded once in a
        # HIP graph, replayed once per step (no launch gaps from the host)
        ref = dst.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(dst, ref), "graph-replayed prefill step differs from the eager step"
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            g.replay()
        e1.record()
        e1.synchronize()
        torch.cuda.synchronize()
        del g
        return e0.elapsed_time(e1) / args.steps

    with torch.no_grad():
        ms_step_eager, (ms_compress, ms_attn) = eager(routed, 3)
        ms_two_eager, (_, ms_route, ms_attn_lists) = eager(two_launch, 4)
        assert torch.isfinite(out.float()).all(), "non-finite prefill output"
        assert torch.equal(out, out2), "routed prefill differs from route + prefill"
        t = torch.arange(T, device="cuda")

        def useful_pairs(sel, n):
            # for each (b, g, t) the allowed keys: every listed block below the
            # own one in full, t%bs+1 keys of the own block when it is listed
            last = torch.gather(sel, -1, (n.to(torch.int64) - 1).clamp(min=0)[..., None])[..., 0]
            own_listed = (last == t // BS).to(torch.int64)
            keys = n.to(torch.int64) * BS - own_listed * (BS - (t % BS + 1))
            return int(keys.sum().item()) * (HQ // HKV)

        pairs = useful_pairs(state["sel"], state["n"])
        ms_step = graphed(routed, out)
        ms_two = graphed(two_launch, out2)
        chunk = {}
        if out3 is not None:
            ms_ch_eager, (_, ms_ch_route, ms_ch_attn) = eager(chunked, 4)
            assert torch.isfinite(out3.float()).all(), "non-finite chunked prefill output"
            csel, cn = sparda.select_chunked(state["ctopk"], B, HKV, T, BS, TOPK)
            cflop = 4 * D * useful_pairs(csel, cn)
            ms_ch = graphed(chunked, out3)
            chunk = {"chunked": {
                "ms_per_step": ms_ch, "tok_s": B * T / (ms_ch * 1e-3), "ms_per_step_eager": ms_ch_eager,
                "route_us": ms_ch_route * 1e3, "attn_us": ms_ch_attn * 1e3,
                "attn_useful_flop": cflop, "attn_tflops": cflop / (ms_ch_attn * 1e-3) / 1e12,
                "attn_frac": cflop / (ms_ch_attn * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}}
        # the dense causal step of the same layer (the reference's dense
        # fallback: layer 0 of every forward), kernel time by events
        dense = {}
        if T == MT:
            ms_dense = events_ms(lambda: sparda.prefill(q, k, v, None, None, BS, out=out2), args.steps, torch)
            dflop = 4 * D * HQ * B * T * (T + 1) // 2
            dense = {"dense_attn_us": ms_dense * 1e3, "dense_attn_tflops": dflop / (ms_dense * 1e-3) / 1e12,
                     "dense_attn_frac": dflop / (ms_dense * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}
    flops = 4 * D * pairs
    tflops = flops / (ms_attn * 1e-3) / 1e12
    # compressor: read K, write the fp32 prototypes; router: read the forecast
    # (bf16, [B,T,Hkv,64]) and the prototypes, write the lists and counts
    nb = (T + BS - 1) // BS
    comp_bytes = B * T * HKV * D * 2 + B * nb * HKV * D * 4
    route_bytes = B * T * HKV * D * 2 + B * nb * HKV * D * 4 + B * HKV * T * (TOPK + 3) * 4
    return {
        "ms_per_step": ms_step,
        "tok_s": B * T / (ms_step * 1e-3),
        "ms_per_step_eager": ms_step_eager,
        "attn_ms": ms_attn,
        "attn_useful_flop": flops,
        "attn_tflops": tflops,
        "compress_us": ms_compress * 1e3,
        "compress_gbs": comp_bytes / (ms_compress * 1e-3) / 1e9,
        "compress_frac": comp_bytes / (ms_compress * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "two_launch_ms_per_step": ms_two,
        "two_launch_ms_per_step_eager": ms_two_eager,
        "two_launch_tok_s": B * T / (ms_two * 1e-3),
        "route_us": ms_route * 1e3,
        "route_gbs": route_bytes / (ms_route * 1e-3) / 1e9,
        "route_frac": route_bytes / (ms_route * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "attn_from_lists_us": ms_attn_lists * 1e3,
        "attn_from_lists_tflops": flops / (ms_attn_lists * 1e-3) / 1e12,
        "dense_causal_flop": 4 * D * HQ * B * T * (T + 1) // 2,
        **dense,
        **chunk,
    }


def bench_decode(args, torch, sparda, synth):
    caches = [synth.decode_inputs(DB, DS, HQ, HKV, D, dtype=torch.bfloat16, seed=1002 + i, device="cuda")
              for i in range(N_CACHES)]
    ws = sparda.DecodeWorkspace("cuda")
    outs = [torch.empty((DB, HQ * D), dtype=torch.bfloat16, device="cuda") for _ in range(N_CACHES)]

    def one(i):
        c = caches[i % N_CACHES]
        sparda.decode(c["q"], c["k_cache"], c["v_cache"], DS, c["forecast"], BS, TOPK, routing="absolute",
                      workspace=ws, out=outs[i % N_CACHES])

    with torch.no_grad():
        for i in range(8):
            one(i)
        torch.cuda.synchronize()
        eager_us = events_ms(lambda: [one(i) for i in range(args.decode_steps)], 1, torch) * 1e3 / args.decode_steps
        # capture the timed steps in one HIP graph (the decode kernels keep no
        # state between calls, so replays need no memset nodes)
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(4):
                one(i)
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(g):
            for i in range(args.decode_steps):
                one(i)
        g.replay()
        torch.cuda.synchronize()
        graph_us = events_ms(g.replay, 3, torch) * 1e3 / args.decode_steps
        # selections -> gathered bytes per step (exact)
        gathered = 0
        for c in caches:
            _, ex = sparda.decode(c["q"], c["k_cache"], c["v_cache"], DS, c["forecast"], BS, TOPK,
                                  routing="absolute", workspace=ws, want_sel=True)
            gathered += int(ex["n_sel"].sum().item()) * BS * D * 2 * 2
        gathered //= N_CACHES
        # check one output against a fresh eager call
        ref = sparda.decode(caches[0]["q"], caches[0]["k_cache"], caches[0]["v_cache"], DS, caches[0]["forecast"],
                            BS, TOPK, routing="absolute", workspace=ws)
        assert torch.equal(ref, outs[0]), "graph replay differs from eager decode"
        # cached prototypes: block sums kept in HBM; one launch recomputes the
        # current block's sums (64 tokens), scores the blocks from the sums,
        # selects and attends in place -- no whole-cache compression. Also
        # timed with the sums update as a separate launch before it.
        nb = DS // BS
        cb = (DS - 1) // BS
        sums = [torch.zeros((DB, nb, HKV, D), dtype=torch.float32, device="cuda") for _ in range(N_CACHES)]
        outs_c = [torch.empty((DB, HQ * D), dtype=torch.bfloat16, device="cuda") for _ in range(N_CACHES)]
        for i, c in enumerate(caches):
            sparda.block_sums(c["k_cache"], 0, DS, BS, sums[i])

        def one_cached(i, separate=False):
            j = i % N_CACHES
            c = caches[j]
            if separate:
                sparda.block_sums(c["k_cache"], cb * BS, DS - cb * BS, BS, sums[j])
            sparda.decode_sums(c["q"], c["k_cache"], c["v_cache"], DS, c["forecast"], sums[j], BS, TOPK,
                               routing="absolute", out=outs_c[j], update_current=not separate)

        def replayed(separate):
            gc = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for i in range(4):
                    one_cached(i, separate)
            torch.cuda.current_stream().wait_stream(side)
            with torch.cuda.graph(gc):
                for i in range(args.decode_steps):
                    one_cached(i, separate)
            gc.replay()
            torch.cuda.synchronize()
            return events_ms(gc.replay, 3, torch) * 1e3 / args.decode_steps

        for i in range(8):
            one_cached(i)
        torch.cuda.synchronize()
        eager_c_us = events_ms(lambda: [one_cached(i) for i in range(args.decode_steps)], 1, torch) * 1e3 / args.decode_steps
        cached_sep_us = replayed(True)
        cached_us = replayed(False)
        # the cached step's selection equals the faithful step's, its output the
        # attention over that selection
        c0 = caches[0]
        _, ex = sparda.decode(c0["q"], c0["k_cache"], c0["v_cache"], DS, c0["forecast"], BS, TOPK,
                              routing="absolute", workspace=ws, want_sel=True)
        o4, s4, n4 = sparda.decode_sums(c0["q"], c0["k_cache"], c0["v_cache"], DS, c0["forecast"], sums[0], BS,
                                        TOPK, routing="absolute", want_sel=True)
        assert torch.equal(s4, ex["sel"]) and torch.equal(n4, ex["n_sel"]), "cached selection differs"
        assert torch.equal(o4, outs_c[0]), "graph-replayed cached step differs from the eager one"
    k_stream = DB * DS * HKV * D * 2
    small = DB * HQ * D * 2 * 2 + DB * HKV * D * 2 + DB * HKV * (DS // BS) * 4 * 2
    total = k_stream + gathered + small
    cached_total = DB * nb * HKV * D * 4 + DB * BS * HKV * D * 2 + gathered + DB * HQ * D * 2 * 2 + DB * HKV * D * 2
    return {
        "us_per_step": graph_us,
        "us_per_step_eager": eager_us,
        "bytes_per_step": total,
        "gbs": total / (graph_us * 1e-6) / 1e9,
        "k_stream_bytes": k_stream,
        "gathered_bytes": gathered,
        "us_per_step_cached_protos": cached_us,
        "us_per_step_cached_protos_eager": eager_c_us,
        "us_per_step_cached_protos_separate_sums": cached_sep_us,
        "cached_bytes_per_step": cached_total,
    }


def bench_offload(args, torch, sparda, synth):
    """12-layer decode at a 32K context with every layer but layer 0 holding its
    KV in a pinned host arena: forecast-routed blocks prefetched while the
    previous layer runs (eagerly on a side stream; replayed from a graph,
    carried by the previous layer's attention launch, on a side stream, or
    serially). Also times the synchronous offload step, the fully GPU-resident
    sparse step, and one layer's attention launch with and without the next
    layer's prefetch inside it."""
    from model.attention import AsyncOffloadedKVCache, KVCache, OffloadedKVCache, PrototypeKVCache
    from model.config import ModelConfig
    from model.model import SparDAResearchModel
    dev = torch.device("cuda")
    W, K = 4, args.offload_steps
    cap = OB_CTX + 8 * (W + K) + 64
    # the fused producer and decode FFN, as the generation leg uses them
    cfg = ModelConfig(n_layer=OB_LAYERS, context_length=cap, block_size=BS, top_k_blocks=TOPK,
                      decode_routing="absolute", attention_backend="async_offload", norm_eps=1e-5,
                      fused_producer=True, fused_ffn=True)
    torch.manual_seed(1004)
    model = SparDAResearchModel(cfg).to(dev, torch.bfloat16).eval()
    res_cfg = ModelConfig(**{**cfg.__dict__, "attention_backend": "hip_sparse"})
    sync_cfg = ModelConfig(**{**cfg.__dict__, "attention_backend": "offload"})
    resident = SparDAResearchModel(res_cfg).to(dev, torch.bfloat16).eval()
    resident.load_state_dict(model.state_dict())
    syncm = SparDAResearchModel(sync_cfg).to(dev, torch.bfloat16).eval()
    syncm.load_state_dict(model.state_dict())

    off_caches = [KVCache(1, cap, HKV, D, dev, torch.bfloat16)] + [
        AsyncOffloadedKVCache(1, cap, HKV, D, dev, torch.bfloat16, block_size=BS) for _ in range(OB_LAYERS - 1)]
    res_caches = [KVCache(1, cap, HKV, D, dev, torch.bfloat16) for _ in range(OB_LAYERS)]
    for li in range(OB_LAYERS):  # the same synthetic context in both cache sets
        for _, k, v in synth.kv_chunks(1, OB_CTX, HKV, D, seed=2000 + li):
            kd, vd = k.to(dev, torch.bfloat16), v.to(dev, torch.bfloat16)
            off_caches[li].update(kd, vd)
            res_caches[li].update(kd, vd)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(1006)
    ids = torch.randint(0, cfg.vocab_size, (12 * (W + K), 1, 1), generator=g).to(dev)
    it = iter(range(ids.shape[0]))

    def run(m, caches, n):
        with torch.no_grad():
            for _ in range(n):
                m(ids[next(it)], kv_caches=caches)

    def timed(m, caches):
        run(m, caches, W)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run(m, caches, K)
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / K

    # async prefetch: device-event overlap on every prefetched layer
    attns = [model.layers[i].attention for i in range(1, OB_LAYERS)]
    for a in attns:
        a.track_overlap = True
    run(model, off_caches, W)
    torch.cuda.synchronize()
    for a in attns:
        a.overlap_stats(reset=True)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    run(model, off_caches, K)
    e1.record()
    e1.synchronize()
    us_async = e0.elapsed_time(e1) * 1e3 / K
    stats = [a.overlap_stats() for a in attns]
    stale = sum(a.stale_prefetches for a in attns)
    tr = sum(s["transfer_ms"] for s in stats) / len(stats)
    ex = sum(s["exposed_ms"] for s in stats) / len(stats)
    fetched = sum(a.prefetched_bytes for a in attns)
    for a in attns:
        a.track_overlap = False
    # same caches, synchronous offload (select + fetch on the compute stream)
    us_sync = timed(syncm, off_caches)
    us_res = timed(resident, res_caches)
    # the fetch as DMA copies (hipMemcpyAsync per run of consecutive blocks;
    # the host waits for the selection once per fetch), async and sync
    for m_ in (model, syncm):
        for layer in m_.layers[1:]:
            layer.attention.fetch_method = sparda.FETCH_DMA
    us_async_dma = timed(model, off_caches)
    us_sync_dma = timed(syncm, off_caches)
    for m_ in (model, syncm):
        for layer in m_.layers[1:]:
            layer.attention.fetch_method = sparda.FETCH_KERNEL

    def graph_step_us(m, caches, reps=50):
        """One decode step captured in a HIP graph at a fixed position (each
        replay re-appends the same token at the same slot); the replayed logits
        must equal an eager step at that position."""
        x = ids[0]
        with torch.no_grad():
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                m(x, kv_caches=caches)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            lens = [c.current_len for c in caches]
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                logits = m(x, kv_caches=caches)["logits"]
            for _ in range(3):
                g.replay()
            torch.cuda.synchronize()
            us = events_ms(g.replay, reps, torch) * 1e3
            got = logits.clone()
            for c, n in zip(caches, lens):
                c.current_len = n
            want = m(x, kv_caches=caches)["logits"]
            torch.cuda.synchronize()
            assert torch.equal(got, want), "graph replay differs from the eager decode step"
        del g
        return us

    # the GPU-resident step replayed from a HIP graph: whole-cache compression
    # every step (KVCache), and cached prototypes (PrototypeKVCache)
    us_res_graph = graph_step_us(resident, res_caches)
    proto_caches = [PrototypeKVCache(1, cap, HKV, D, dev, torch.bfloat16, block_size=BS) for _ in range(OB_LAYERS)]
    with torch.no_grad():
        for pc, rc in zip(proto_caches, res_caches):
            pc.update(rc.k[:, :rc.current_len], rc.v[:, :rc.current_len])
    us_proto_eager = timed(resident, proto_caches)
    us_proto_graph = graph_step_us(resident, proto_caches)
    del proto_caches

    # the offloaded step replayed from a HIP graph (GraphDecoder over the same
    # host arenas, positions in device memory): the prefetch of layer L+1
    # carried by layer L's attention launch (the default), on a side stream
    # under layer L's attention + FFN, and on the compute stream (no overlap)
    from model.decode_graph import GraphDecoder

    # the three decoders are recorded first, then timed in alternating rounds
    # of S steps (median over the rounds), so that a drift of the host link
    # or clocks during the run affects the three alike
    R, S = 8, max(1, K // 8)
    decs = {name: GraphDecoder(model, 1, cap, caches=off_caches, overlap=m)
            for name, m in (("fused", "fused"), ("side", True), ("serial", False))}
    rounds = {name: [] for name in decs}
    with torch.no_grad():
        for gd in decs.values():
            for _ in range(W):
                gd.step(ids[next(it)])
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(R):
            for name, gd in decs.items():
                e0.record()
                for _ in range(S):
                    gd.step(ids[next(it)])
                e1.record()
                e1.synchronize()
                rounds[name].append(e0.elapsed_time(e1) * 1e3 / S)
    del decs
    med = {name: sorted(v)[len(v) // 2] for name, v in rounds.items()}
    us_off_graph, us_off_graph_side, us_off_graph_serial = med["fused"], med["side"], med["serial"]

    # one layer's launches at this context (HIP events on the launch stream):
    # layer 1's attention over its fetched blocks alone, layer 2's prefetch
    # (selection + host-link copy) as launches of their own, and layer 1's
    # attention launch carrying layer 2's prefetch
    c1, c2 = off_caches[1], off_caches[2]
    L = c1.current_len
    pos = torch.full((1,), L, dtype=torch.int64, device=dev)
    gq = torch.Generator().manual_seed(1007)
    q1 = torch.randn(1, HQ, D, generator=gq).to(dev, torch.bfloat16)
    kn1 = torch.randn(1, HKV, D, generator=gq).to(dev, torch.bfloat16)
    vn1 = torch.randn(1, HKV, D, generator=gq).to(dev, torch.bfloat16)
    f1 = torch.randn(1, HKV, D, generator=gq).to(dev, torch.bfloat16)
    bufs = [dict(sel=torch.empty((1, HKV, TOPK + 2), dtype=torch.int32, device=dev),
                 n=torch.empty((1, HKV), dtype=torch.int32, device=dev),
                 k=torch.empty((1, HKV, TOPK + 2, BS, D), dtype=torch.bfloat16, device=dev),
                 v=torch.empty((1, HKV, TOPK + 2, BS, D), dtype=torch.bfloat16, device=dev)) for _ in range(2)]

    def prefetch_into(c, bq):
        sparda.select_decode_at(f1, c.block_sums(BS), pos, cap, BS, TOPK, routing="absolute", sel=bq["sel"],
                                n_sel=bq["n"], lookahead=True)
        c.arena.fetch_at(bq["sel"], bq["n"], BS, pos, bq["k"], bq["v"])

    prefetch_into(c1, bufs[0])
    spec = dict(arena=c2.arena, forecast=f1, block_sums=c2.block_sums(BS), top_k=TOPK, routing="absolute",
                sel=bufs[1]["sel"], n_sel=bufs[1]["n"], k_dst=bufs[1]["k"], v_dst=bufs[1]["v"])

    def attend(carry=None):
        sparda.decode_at(q1, bufs[0]["k"], bufs[0]["v"], pos, BS, bufs[0]["sel"], bufs[0]["n"], max_len=cap,
                         compact=True, k_new=kn1, v_new=vn1, prefetch=carry)

    t_attn = events_ms(attend, 50, torch) * 1e3
    t_pf = events_ms(lambda: prefetch_into(c2, bufs[1]), 50, torch) * 1e3
    t_carry = events_ms(lambda: attend(spec), 50, torch) * 1e3
    carried = {
        "attention_us": round(t_attn, 2),
        "prefetch_separate_us": round(t_pf, 2),
        "attention_carrying_prefetch_us": round(t_carry, 2),
        "hidden_us": round(t_attn + t_pf - t_carry, 2),
        "overlap": round(min(1.0, max(0.0, 1.0 - (t_carry - t_attn) / t_pf)), 4) if t_pf > 0 else None,
    }
    # host link: one 256 MiB pinned host -> device copy
    hb = torch.empty(256 << 20, dtype=torch.uint8).pin_memory()
    db = torch.empty_like(hb, device=dev)
    db.copy_(hb, non_blocking=True)
    torch.cuda.synchronize()
    link_ms = events_ms(lambda: db.copy_(hb, non_blocking=True), 5, torch)
    del hb, db
    per_layer = fetched / len(attns)
    return {
        "workload": f"decode with offloaded KV: {OB_LAYERS} layers, B=1, context {OB_CTX} (512 blocks of 64), "
                    f"bf16 KV [32768,4,64] per layer in pinned host memory for layers 1..{OB_LAYERS - 1} "
                    "(layer 0 GPU-resident), top-8 + sink + current blocks prefetched per layer (eager: on a side "
                    "stream; replayed: carried by the previous layer's append and attention launches, or on a side "
                    "stream, or serial); fused producer and decode FFN; step = one token through the 12-layer model "
                    "incl. LM head",
        "us_per_step_async": round(us_async, 1),
        "us_per_step_sync": round(us_sync, 1),
        "us_per_step_async_dma": round(us_async_dma, 1),
        "us_per_step_sync_dma": round(us_sync_dma, 1),
        "us_per_step_gpu_resident": round(us_res, 1),
        "us_per_step_gpu_resident_graph": round(us_res_graph, 1),
        "us_per_step_cached_prototypes": round(us_proto_eager, 1),
        "us_per_step_cached_prototypes_graph": round(us_proto_graph, 1),
        "us_per_step_async_graph": round(us_off_graph, 1),
        "us_per_step_async_graph_side_stream": round(us_off_graph_side, 1),
        "us_per_step_async_graph_serial_prefetch": round(us_off_graph_serial, 1),
        "async_graph_rounds_us": {name: [round(x, 1) for x in v] for name, v in rounds.items()},
        "carried_prefetch_one_layer": carried,
        "steps": K,
        "overlap": round(1.0 - ex / tr, 4) if tr > 0 else None,
        "transfer_us_per_layer": round(tr * 1e3, 2),
        "exposed_us_per_layer": round(ex * 1e3, 2),
        "h2d_bytes_per_step": int(fetched),
        "h2d_gbs_per_layer": round(per_layer / (tr * 1e-3) / 1e9, 2) if tr > 0 else None,
        "host_link_gbs": round((256 << 20) / (link_ms * 1e-3) / 1e9, 2),
        "stale_prefetches": stale,
    }


def bench_generate(args, torch, sparda, synth, batch=1):
    """Greedy generation after a 16384-token prompt with the 12-layer model of
    bench_model (fused producer, cached prototypes, absolute-position routing,
    B=1, then B=8 sequences decoded together): per-step time of the eager
    cached decode loop (host-driven, one launch sequence issued per token) and
    of GraphDecoder (one HIP graph replay per step, positions read from device
    memory). Both loops start from the same prefill; their generated tokens
    must agree."""
    from model.attention import PrototypeKVCache
    from model.config import ModelConfig
    from model.decode_graph import GraphDecoder
    from model.model import SparDAResearchModel
    dev = torch.device("cuda")
    G, W = args.generate_steps, 8
    cap = MT + G + W + 64
    cfg = ModelConfig(n_layer=12, context_length=cap, block_size=BS, top_k_blocks=TOPK,
                      attention_backend="hip_sparse", norm_eps=1e-5, fused_producer=True, fused_ffn=True,
                      decode_routing="absolute")
    torch.manual_seed(1007)
    model = SparDAResearchModel(cfg).to(dev, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(1007)
    prompt = torch.randint(0, cfg.vocab_size, (batch, MT), generator=g).to(dev)

    def loop(first_logits, step, n):
        toks, logits = [], first_logits
        for _ in range(n):
            nxt = torch.argmax(logits, dim=-1, keepdim=True)
            toks.append(nxt)
            logits = step(nxt)
        return toks, logits

    def timed(step, first_logits):
        toks, logits = loop(first_logits, step, W)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        more, _ = loop(logits, step, G)
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / G, torch.cat(toks + more, dim=1)

    with torch.no_grad():
        caches = [PrototypeKVCache(batch, cap, cfg.n_kv_head, cfg.head_dim, dev, torch.bfloat16, block_size=BS)
                  for _ in range(cfg.n_layer)]
        first = model(prompt, kv_caches=caches)["logits"][:, -1]
        us_eager, toks_eager = timed(lambda t: model(t, kv_caches=caches)["logits"][:, -1], first)
        del caches
        gd = GraphDecoder(model, batch, cap)
        first = gd.prefill(prompt)
        us_graph, toks_graph = timed(gd.step, first)
        torch.cuda.synchronize()
    assert torch.equal(toks_eager, toks_graph), "graph-replayed generation differs from the eager loop"
    del gd, model
    torch.cuda.empty_cache()
    if batch != 1:
        return {"us_per_step_eager": round(us_eager, 1), "us_per_step_graph": round(us_graph, 1),
                "tok_s_graph": round(batch * 1e6 / us_graph, 1)}
    b8 = bench_generate(args, torch, sparda, synth, batch=8)
    return {
        "workload": f"greedy generation of {G} tokens after a {MT}-token prompt, 12-layer model of "
                    "model_forward (fused producer and FFN, block sums kept in HBM, top-8 + sink + current, "
                    "absolute-position routing), bf16; step = one token per sequence through all layers "
                    "incl. LM head; B=1, and B=8 sequences decoded together (*_b8)",
        "us_per_token_eager": round(us_eager, 1),
        "us_per_token_graph": round(us_graph, 1),
        "tok_s_graph": round(1e6 / us_graph, 1),
        "us_per_step_eager_b8": b8["us_per_step_eager"],
        "us_per_step_graph_b8": b8["us_per_step_graph"],
        "tok_s_graph_b8": b8["tok_s_graph"],
        "tokens": G,
        "tokens_agree": True,
    }


def bench_model(args, torch, sparda, synth, fused=False):
    """12-layer forward of the model at B=1, T=16384 (bf16 weights from the
    model's N(0, 0.02) init, vocab 32000 tied, d 768, 12/4 heads, SwiGLU 2048;
    at this length the chunked path in every layer: layer 0 the static
    window, layers 1..11 routed per query block with layer L's forecast
    routing layer L+1), token ids uniform in [0, 32000). Reports
    tok/s of the whole forward (embeddings to logits) and the time of each
    layer's attention (projections + RoPE + compress + routed attention +
    output projection), from HIP events recorded around the attention modules."""
    from model.config import ModelConfig
    from model.model import SparDAResearchModel
    dev = torch.device("cuda")
    cfg = ModelConfig(n_layer=12, context_length=MT, block_size=BS, top_k_blocks=TOPK,
                      attention_backend="hip_sparse", norm_eps=1e-5, fused_producer=fused)
    torch.manual_seed(1003)
    model = SparDAResearchModel(cfg).to(dev, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(1003)
    ids = torch.randint(0, cfg.vocab_size, (1, MT), generator=g).to(dev)
    starts, ends = [], []
    hooks = []
    # per-layer attention events (the fused producer enters the attention past
    # its forward hooks: only the whole forward is timed then)
    for layer in ([] if fused else model.layers):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        starts.append(e0)
        ends.append(e1)
        hooks.append(layer.attention.register_forward_pre_hook(lambda m, a, e=e0: e.record()))
        hooks.append(layer.attention.register_forward_hook(lambda m, a, o, e=e1: e.record()))
    runs = 3
    with torch.no_grad():
        model(ids)
        torch.cuda.synchronize()
        per_layer = [0.0] * len(starts)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        total = 0.0
        for _ in range(runs):
            t0.record()
            model(ids)
            t1.record()
            t1.synchronize()
            total += t0.elapsed_time(t1)
            for i in range(len(per_layer)):
                per_layer[i] += starts[i].elapsed_time(ends[i])
    for h in hooks:
        h.remove()
    ms = total / runs
    attn = [x / runs for x in per_layer]
    del model
    torch.cuda.empty_cache()
    if not fused:
        fz = bench_model(args, torch, sparda, synth, fused=True)
    return {
        "workload": f"12-layer forward, B=1, T={MT}, bf16 (d 768, 12/4 heads, head dim 64, SwiGLU 2048, "
                    "vocab 32000 tied, block 64, top-8); past 8192 tokens every layer takes the chunked "
                    "path (one list per 64-token query block, cut to 10 blocks): layer 0 the static window, "
                    "layers 1-11 routed by the previous layer's forecast; embeddings to logits",
        "ms_per_forward": round(ms, 3),
        "tok_s": round(MT / (ms * 1e-3), 1),
        "attention_ms_per_layer": [round(x, 3) for x in attn],
        "attention_fraction": round(sum(attn) / ms, 4) if attn else None,
        "runs": runs,
        **({} if fused else {"ms_per_forward_fused_producer": fz["ms_per_forward"],
                             "tok_s_fused_producer": fz["tok_s"]}),
    }


def bench_producer(args, torch, sparda, synth):
    """The attention inputs of one layer at the prefill workload (B=4, T=4096,
    d 768): RMSNorm + q / k / v / forecast projections + RoPE, fused (one
    kernel) against the unfused sequence of the reference's modules (RMSNorm,
    four bf16 linears, rotate-half RoPE)."""
    from model.norm import RMSNorm
    from model.rope import apply_rope, rope_tables
    dev = torch.device("cuda")
    C, NQ, NKV, NF = HQ * D, HQ * D, HKV * D, HKV * D
    g = torch.Generator().manual_seed(1005)
    x = torch.randn(PB, PT, C, generator=g).to(dev, torch.bfloat16)
    ws = [(0.02 * torch.randn(n, C, generator=g)).to(dev, torch.bfloat16) for n in (NQ, NKV, NKV, NF)]
    norm = RMSNorm(C, eps=1e-5).to(dev, torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_((1.0 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16))
    cos, sin = (t.to(dev) for t in rope_tables(D, PT))
    w_fold = (torch.cat([w.float() for w in ws]) * norm.weight.float()[None, :]).to(torch.bfloat16).contiguous()

    def unfused():
        h = norm(x)
        q = torch.nn.functional.linear(h, ws[0]).view(PB, PT, HQ, D)
        k = torch.nn.functional.linear(h, ws[1]).view(PB, PT, HKV, D)
        v = torch.nn.functional.linear(h, ws[2]).view(PB, PT, HKV, D)
        f = torch.nn.functional.linear(h, ws[3]).view(PB, PT, HKV, D)
        return apply_rope(q, cos, sin), apply_rope(k, cos, sin), v, f

    def fused():
        return sparda.produce(x, w_fold, NQ, NKV, NF, 1e-5, cos, sin)

    with torch.no_grad():
        for _ in range(3):
            unfused()
            fused()
        torch.cuda.synchronize()
        us_unfused = events_ms(unfused, 20, torch) * 1e3
        us_fused = events_ms(fused, 20, torch) * 1e3
        a, b = unfused(), fused()
        err = max(float((x1.float() - x2.float()).abs().max()) for x1, x2 in zip(a, b))
    flop = 2.0 * PB * PT * (NQ + 2 * NKV + NF) * C
    return {
        "workload": f"RMSNorm + q/k/v/forecast projections + RoPE of one layer, B={PB} T={PT} d={C} "
                    f"(N = {NQ}+{NKV}+{NKV}+{NF}), bf16",
        "us_fused": round(us_fused, 2),
        "us_unfused_torch": round(us_unfused, 2),
        "fused_tflops": round(flop / (us_fused * 1e-6) / 1e12, 1),
        "max_abs_vs_unfused": round(err, 4),
    }


def bench_teacher(args, torch, sparda, synth):
    """Routing-quality teacher at the prefill workload (B=4, T=4096, 12/4
    heads): per-block dense attention mass from q and k in one kernel, against
    the reference's way of getting it (materialised bf16 softmax weights
    [4,12,4096,4096], then TeacherBlockSelector's view / mean / pad / sum)."""
    from model.forecast import TeacherBlockSelector
    x = synth.prefill_inputs(PB, PT, HQ, HKV, D, dtype=torch.bfloat16, seed=1001, device="cuda")
    q, k = x["q"], x["k"]
    sel = TeacherBlockSelector(block_size=BS, num_queries_per_kv=HQ // HKV)
    R = HQ // HKV
    mask = torch.full((PT, PT), float("-inf"), device="cuda").triu(1).to(torch.bfloat16)

    def materialised():
        qh = q.transpose(1, 2)
        kt = k.repeat_interleave(R, dim=2).permute(0, 2, 3, 1).contiguous()
        w = torch.softmax(torch.matmul(qh, kt) * (1.0 / D ** 0.5) + mask, dim=-1)
        return sel(w, TOPK)

    with torch.no_grad():
        mass = sparda.teacher_block_mass(q, k, BS)
        ref = materialised()
        torch.cuda.synchronize()
        err = float((mass - ref[0].float()).abs().max())
        us_kernel = events_ms(lambda: sparda.teacher_block_mass(q, k, BS), 10, torch) * 1e3
        us_mat = events_ms(materialised, 3, torch) * 1e3
    flop = 2 * (4.0 * D * PB * HQ * PT * (PT + 1) / 2)  # QK^T over the causal pairs, two passes
    return {
        "workload": f"teacher block mass, B={PB} T={PT} Hq={HQ} Hkv={HKV} D={D} block={BS}, causal, bf16",
        "us_kernel": round(us_kernel, 1),
        "us_materialised_torch": round(us_mat, 1),
        "kernel_tflops": round(flop / (us_kernel * 1e-6) / 1e12, 1),
        "max_abs_vs_materialised": round(err, 5),
    }


def pmc_workload(args, torch, sparda, synth):
    """Short eager run for hardware-counter passes: at B=4 T=4096, then at B=1
    T=16384, three prefill steps (compress + routed prefill) and one step of
    the three-launch form (compress, router, prefill from its lists); then one
    dense causal prefill at B=1 T=16384 (no lists) and one step of the chunked
    path there (compress, non-causal router, prefill_chunked); decode steps and
    a plain device copy of COPY_BYTES (the calibration of FETCH_SIZE /
    WRITE_SIZE). Counter values are per dispatch, in this order."""
    x = synth.prefill_inputs(PB, PT, HQ, HKV, D, dtype=torch.bfloat16, seed=1001, device="cuda")
    x16 = synth.prefill_inputs(1, MT, HQ, HKV, D, dtype=torch.bfloat16, seed=1003, device="cuda")
    c = synth.decode_inputs(DB, DS, HQ, HKV, D, dtype=torch.bfloat16, seed=1002, device="cuda")
    ws = sparda.DecodeWorkspace("cuda")
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    with torch.no_grad():
        for xs in (x, x16):
            for _ in range(3):
                protos = sparda.compress(xs["k"], BS)
                sparda.prefill_routed(xs["q"], xs["k"], xs["v"], xs["forecast"], protos, BS, TOPK)
            protos = sparda.compress(xs["k"], BS)
            _, _, sel, n_sel = sparda.route(xs["forecast"], protos, BS, TOPK, want_topk=False, want_sel=True)
            sparda.prefill(xs["q"], xs["k"], xs["v"], sel, n_sel, BS)
        sparda.prefill(x16["q"], x16["k"], x16["v"], None, None, BS)
        protos = sparda.compress(x16["k"], BS)
        topk = sparda.route(x16["forecast"], protos, BS, TOPK, causal=False)[0]
        sparda.prefill_chunked(x16["q"], x16["k"], x16["v"], topk, BS, TOPK)
        for _ in range(3):
            sparda.decode(c["q"], c["k_cache"], c["v_cache"], DS, c["forecast"], BS, TOPK, routing="absolute",
                          workspace=ws)
        for _ in range(3):
            dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_bytes": COPY_BYTES}


def cpu_info():
    """Host CPU model (/proc/cpuinfo, what lscpu's "Model name" shows), the
    physical cores and the cores this process may run on."""
    model, cores = None, set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as fh:
            for ln in fh:
                k, _, v = ln.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"model": model, "physical_cores": len(cores) or None, "os_cpu_count": os.cpu_count(),
            "usable_cpus": usable}


def cpu_timed(fn, warmup=3, runs=10):
    """The reference's latency protocol (evaluation/latency.py:30-31,69-74):
    `warmup` untimed calls, then `runs` calls timed with perf_counter;
    returns the median and the spread in seconds."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    mid = len(ts) // 2
    med = ts[mid] if len(ts) % 2 else 0.5 * (ts[mid - 1] + ts[mid])
    return med, ts[0], ts[-1]


def _thread_counts(args, torch):
    n = args.cpu_threads or torch.get_num_threads()
    return [n, 1] if n != 1 else [1]


def cpu_decode_baseline(args, torch, synth, info):
    """The reference's decode step restated op for op (oracle/reference_path.py:
    whole-cache recompression, selection, topk compaction, gather, masked SDPA)
    on the host cores, at the decode workload (B=8, 16K cache, bf16), routed
    like the GPU leg (absolute-position causal mask; the reference's row-0 mask
    is the same operations on another mask row). N threads and 1 thread,
    warm-up 3 / runs 20 of 16 steps each, median per step, with the fastest
    and slowest run beside it."""
    from oracle import reference_path as R
    x = synth.decode_inputs(DB, DS, HQ, HKV, D, dtype=torch.bfloat16, seed=1002)
    q = x["q"][:, :, None, :]
    k, v = x["k_cache"].transpose(1, 2), x["v_cache"].transpose(1, 2)
    f = x["forecast"][:, None]
    steps = 16
    legs = {}
    with torch.no_grad():
        for n in _thread_counts(args, torch):
            torch.set_num_threads(n)
            med, lo, hi = cpu_timed(lambda: [R.sparse_decode(q, k, v, DS, f, BS, TOPK, routing="absolute")
                                             for _ in range(steps)], runs=20)
            legs[n] = (med / steps, lo / steps, hi / steps)
    torch.set_num_threads(max(legs))
    n = max(legs)
    out = {"value": round(legs[n][0] * 1e6, 1), "unit": "us/step", "cores": n, "kind": "port",
           "sample": f"the decode workload (B=8, 16K cache, bf16) through the reference's decode step restated "
                     f"op for op in PyTorch (whole-cache recompression, absolute-position routing as the GPU "
                     f"leg, topk compaction, gather, masked SDPA); warm-up 3, median of 20 runs of {steps} "
                     f"steps; torch threads={n}",
           "min_us": round(legs[n][1] * 1e6, 1), "max_us": round(legs[n][2] * 1e6, 1), "cpu": info}
    if 1 in legs and n != 1:
        out["value_1_thread"] = round(legs[1][0] * 1e6, 1)
    return out


def cpu_chunked_baseline(args, torch, synth, info):
    """The reference's chunked-gather prefill (its path past 8192 tokens)
    restated op for op (oracle/reference_path.py) on the host cores, at the
    16K leg's shape (B=1, T=16384, one layer): compress, then per 64-token
    query block the non-causal selector, the mask and its top-k cut, the
    gather and SDPA. Warm-up 1, runs 3, median (each run is one whole layer)."""
    from oracle import reference_path as R
    x = synth.prefill_inputs(1, MT, HQ, HKV, D, dtype=torch.bfloat16, seed=1003)
    q, k, v = (x[n].transpose(1, 2) for n in ("q", "k", "v"))
    f = x["forecast"]
    n = max(_thread_counts(args, torch))
    torch.set_num_threads(n)
    with torch.no_grad():
        med, lo, hi = cpu_timed(lambda: R.chunked_prefill(q, k, v, f, BS, TOPK), warmup=1, runs=3)
    return {"value": round(MT / med, 1), "unit": "tok/s", "cores": n, "kind": "port",
            "sample": f"one layer at B=1, T={MT} (bf16) through the reference's chunked-gather path restated "
                      f"op for op in PyTorch (a loop over the 256 query blocks: selector, mask, top-k cut, gather, "
                      f"SDPA); warm-up 1, median of 3 runs, {med:.3f} s/run (min {lo:.3f}, max {hi:.3f}); "
                      f"torch threads={n}",
            "cpu": info}


def cpu_baseline(args, torch, synth, info):
    """Reference prefill path restated op for op (oracle/reference_path.py) on
    the host cores: the full workload (B=4, T=4096) on N threads; on 1 thread
    one sequence of it (B=1, T=4096, the same per-sequence work). Warm-up 3 /
    runs 10, median."""
    from oracle import reference_path as R
    x = synth.prefill_inputs(PB, PT, HQ, HKV, D, dtype=torch.bfloat16, seed=1001)
    q, k, v = (x[n].transpose(1, 2) for n in ("q", "k", "v"))
    f = x["forecast"]
    legs = {}
    counts = _thread_counts(args, torch)  # once: it reads torch's thread count, which the loop changes
    with torch.no_grad():
        for n in counts:
            torch.set_num_threads(n)
            b = PB if n == max(counts) else 1
            med, lo, hi = cpu_timed(lambda: R.sparse_prefill(q[:b], k[:b], v[:b], f[:b], BS, TOPK))
            legs[n] = (b * PT / med, b, med, lo, hi)
    n = max(legs)
    torch.set_num_threads(n)
    out = {"value": round(legs[n][0], 1), "unit": "tok/s", "cores": n, "kind": "port",
           "sample": f"the full prefill workload (B={PB}, T={PT}, bf16) through the reference's masked-SDPA "
                     f"path restated op for op in PyTorch (O(T^2) masks + SDPA); warm-up 3, median of 10 runs, "
                     f"{legs[n][2]:.3f} s/run (min {legs[n][3]:.3f}, max {legs[n][4]:.3f}); torch threads={n}",
           "cpu": info}
    if 1 in legs and n != 1:
        out["value_1_thread"] = round(legs[1][0], 1)
        out["sample_1_thread"] = f"one sequence (B=1, T={PT}), warm-up 3, median of 10 runs, {legs[1][2]:.3f} s/run"
    return out


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the sparse attention layer runs on a single MI355X here; "
              "multi-GPU figures are not produced (use --gpus 1).", file=sys.stderr)
        sys.exit(2)
    import torch
    import sparda
    from sparda import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    sparda.load()
    if args.only != "all":
        fn = {"prefill": bench_prefill, "decode": bench_decode, "offload": bench_offload,
              "prefill16k": lambda *a: bench_prefill(*a, B=1, T=MT, seed=1003),
              "model": bench_model, "producer": bench_producer, "teacher": bench_teacher,
              "generate": bench_generate, "pmc": pmc_workload}[args.only]
        r = fn(args, torch, sparda, synth)
        print(json.dumps({args.only: {k: v for k, v in r.items() if isinstance(v, (int, float, str, list, dict))}}),
              flush=True)
        return
    log("prefill workload")
    pre = bench_prefill(args, torch, sparda, synth)
    log(f"prefill: {pre['ms_per_step']:.3f} ms/step, attention {pre['attn_ms']*1e3:.1f} us "
        f"({pre['attn_tflops']:.1f} TFLOP/s useful)")
    log(f"prefill at T={MT} (one layer of the 12-layer forward's shape)")
    p16 = bench_prefill(args, torch, sparda, synth, B=1, T=MT, seed=1003)
    log(f"prefill 16K: {p16['ms_per_step']:.3f} ms/step, attention {p16['attn_ms']*1e3:.1f} us "
        f"({p16['attn_tflops']:.1f} TFLOP/s useful); chunked path {p16['chunked']['ms_per_step']:.3f} ms/step "
        f"(route {p16['chunked']['route_us']:.1f} us, lists + attention {p16['chunked']['attn_us']:.1f} us)")
    log("prefill with the reference's default block configuration (32-key blocks, top-4)")
    p32 = bench_prefill(args, torch, sparda, synth, BS=32, TOPK=4)
    log(f"prefill bs=32 k=4: {p32['ms_per_step']:.3f} ms/step, attention {p32['attn_ms']*1e3:.1f} us")
    log("decode workload")
    dec = bench_decode(args, torch, sparda, synth)
    log(f"decode: {dec['us_per_step']:.2f} us/step ({dec['gbs']:.0f} GB/s), eager {dec['us_per_step_eager']:.2f}; "
        f"cached prototypes {dec['us_per_step_cached_protos']:.2f} us/step")
    log("offload workload")
    off = bench_offload(args, torch, sparda, synth)
    log(f"offload: async {off['us_per_step_async']:.1f} us/step, sync {off['us_per_step_sync']:.1f}, "
        f"resident {off['us_per_step_gpu_resident']:.1f} (graph {off['us_per_step_gpu_resident_graph']:.1f}; "
        f"cached prototypes {off['us_per_step_cached_prototypes']:.1f}, graph "
        f"{off['us_per_step_cached_prototypes_graph']:.1f}); async graph {off['us_per_step_async_graph']:.1f} "
        f"(serial prefetch {off['us_per_step_async_graph_serial_prefetch']:.1f}); overlap {off['overlap']}, "
        f"transfer {off['transfer_us_per_layer']} us/layer, link {off['host_link_gbs']} GB/s; DMA fetch: async "
        f"{off['us_per_step_async_dma']:.1f}, sync {off['us_per_step_sync_dma']:.1f}")
    log("12-layer forward workload")
    mdl = bench_model(args, torch, sparda, synth)
    log(f"model: {mdl['ms_per_forward']:.2f} ms per {MT}-token forward ({mdl['tok_s']:.0f} tok/s), "
        f"attention {100 * mdl['attention_fraction']:.1f}% (layer 0 window {mdl['attention_ms_per_layer'][0]:.2f} ms, "
        f"sparse layers {sum(mdl['attention_ms_per_layer'][1:]) / 11:.2f} ms each); fused producer "
        f"{mdl['ms_per_forward_fused_producer']:.2f} ms ({mdl['tok_s_fused_producer']:.0f} tok/s)")
    log("graph-replayed generation")
    gen = bench_generate(args, torch, sparda, synth)
    log(f"generate: eager {gen['us_per_token_eager']:.1f} us/token, graph {gen['us_per_token_graph']:.1f} us/token; "
        f"B=8 graph {gen['us_per_step_graph_b8']:.1f} us/step ({gen['tok_s_graph_b8']:.0f} tok/s)")
    log("fused producer")
    prod = bench_producer(args, torch, sparda, synth)
    log(f"producer: fused {prod['us_fused']:.1f} us ({prod['fused_tflops']:.0f} TFLOP/s), "
        f"unfused torch {prod['us_unfused_torch']:.1f} us")
    log("routing-quality teacher")
    tch = bench_teacher(args, torch, sparda, synth)
    log(f"teacher: kernel {tch['us_kernel']:.1f} us ({tch['kernel_tflops']:.0f} TFLOP/s), materialised torch "
        f"{tch['us_materialised_torch']:.1f} us")
    cpu = cpu_dec = cpu_ch = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        info = cpu_info()
        cpu = cpu_baseline(args, torch, synth, info)
        log(f"cpu: {cpu['value']:.1f} tok/s on {cpu['cores']} threads, {cpu.get('value_1_thread')} on 1 "
            f"({info['model']})")
        cpu_dec = cpu_decode_baseline(args, torch, synth, info)
        log(f"cpu decode: {cpu_dec['value']:.1f} us/step on {cpu_dec['cores']} threads, "
            f"{cpu_dec.get('value_1_thread')} on 1")
        cpu_ch = cpu_chunked_baseline(args, torch, synth, info)
        log(f"cpu chunked prefill at T={MT}: {cpu_ch['value']:.1f} tok/s on {cpu_ch['cores']} threads")

    traffic = load_traffic()
    ch16 = p16["chunked"]
    t_attn = traffic.get("prefill_attention")
    t_dec = traffic.get("decode_step")
    line = {
        "metric": METRIC,
        "value": round(pre["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "sparse prefill layer: B=4 T=4096 Hq=12 Hkv=4 D=64 block=64 (64 blocks) "
                               "top-k=8 causal, bf16; step = compress + routed block-sparse MFMA prefill (the "
                               "attention kernel routes its own query windows)",
                   "global_batch": PB, "seq_len": PT, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": round(pre["attn_tflops"], 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(pre["attn_tflops"] / PEAK_BF16_TFLOPS, 4),
                     "traffic": t_attn},
        "cpu_baseline": cpu,
        "prefill_detail": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in pre.items()},
        "prefill_16k": {
            "workload": f"the same layer at B=1, T={MT} (256 blocks, top-8), the attention shape of one layer of "
                        "the 12-layer forward, on the path the reference and the backend take past 8192 tokens: "
                        "compress + every row's non-causal top-k + one launch that builds each 64-token query "
                        "block's list (sink + own + the union of its rows' picks, cut to 10 blocks) and attends "
                        "causally over it on the matrix cores; HIP graph replay. per_token_rule: the same layer "
                        "under the per-token rule (compress + routed prefill)",
            "ms_per_step": round(ch16["ms_per_step"], 4),
            "tok_s": round(ch16["tok_s"], 1),
            "roofline": {"bound": "mfma", "achieved": round(ch16["attn_tflops"], 2), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ch16["attn_tflops"] / PEAK_BF16_TFLOPS, 4),
                         "traffic": traffic.get("prefill_chunked_16k")},
            **{k: (round(v, 4) if isinstance(v, float) else v) for k, v in ch16.items()
               if k not in ("ms_per_step", "tok_s")},
            "cpu_baseline": cpu_ch,
            "per_token_rule": {
                "ms_per_step": round(p16["ms_per_step"], 4),
                "tok_s": round(p16["tok_s"], 1),
                "roofline": {"bound": "mfma", "achieved": round(p16["attn_tflops"], 2), "peak": PEAK_BF16_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(p16["attn_tflops"] / PEAK_BF16_TFLOPS, 4),
                             "traffic": traffic.get("prefill_attention_16k")},
                **{k: (round(v, 4) if isinstance(v, float) else v) for k, v in p16.items()
                   if k not in ("ms_per_step", "tok_s", "chunked")}},
        },
        "prefill_block32": {
            "workload": f"the prefill layer at B={PB}, T={PT} with the reference's default block configuration "
                        "(configs/base.yaml: 32-key blocks, top-4; 128 blocks), same step",
            "ms_per_step": round(p32["ms_per_step"], 4),
            "tok_s": round(p32["tok_s"], 1),
            "attn_us": round(p32["attn_ms"] * 1e3, 1),
            "attn_tflops": round(p32["attn_tflops"], 2),
            "attn_useful_flop": p32["attn_useful_flop"],
        },
        "decode": {
            "workload": "decode step @16K: B=8, KV cache [8,16384,4,64] bf16, 256 blocks, top-8 + sink + "
                        "current, absolute-position routing; step = whole-cache compress + route + split-K "
                        "attention + combine; 4 rotating caches; HIP graph replay",
            "us_per_step": round(dec["us_per_step"], 3),
            "us_per_step_eager": round(dec["us_per_step_eager"], 3),
            "steps": args.decode_steps,
            "roofline": {"bound": "hbm", "achieved": round(dec["gbs"], 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(dec["gbs"] / PEAK_HBM_GBS, 4), "traffic": t_dec},
            "cpu_baseline": cpu_dec,
            "bytes_per_step": dec["bytes_per_step"],
            "k_stream_bytes": dec["k_stream_bytes"],
            "gathered_bytes": dec["gathered_bytes"],
            "cached_prototypes": {
                "workload": "the same step with fp32 block sums kept in HBM: one launch recomputes the current "
                            "block's sums, selects from the sums and attends in place (no whole-cache "
                            "compression); *_separate_sums: the sums update as a launch of its own",
                "us_per_step": round(dec["us_per_step_cached_protos"], 3),
                "us_per_step_eager": round(dec["us_per_step_cached_protos_eager"], 3),
                "us_per_step_separate_sums": round(dec["us_per_step_cached_protos_separate_sums"], 3),
                "bytes_per_step": dec["cached_bytes_per_step"],
            },
        },
        "offload": off,
        "model_forward": mdl,
        "generate": gen,
        "producer": prod,
        "teacher": tch,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
