"""Benchmark of the DSA decode hot path on one MI355X.

Default workload ("C3"): DeepSeek-V3.2-shape decode
at 131072-token context, batch 1, one TP-8 share (16 attention heads, the
full 64x128 indexer), two consecutive layers under the MLI lag schedule --
layer L attends layer L-1's top-2048 while layer L's indexer scan and top-k
run concurrently -- captured as one hipGraph.  Each layer is ONE launch of
the fused decode kernel (attention workgroups and indexer-scan/top-k
workgroups side by side in one grid).  A step is one replay of that graph
(2 layers).  Inputs are synthetic N(0,1) (fp8 caches, seeded random page
table of 64-token pages) and resident in HBM before timing starts.

Prints ONE JSON line.  value = microseconds per decode layer (lower is
better).  Extra fields: tokens/s, the standalone indexer-scan GB/s, the MLI
hidden fraction, the roofline of the dominant (and only) kernel of the timed
region -- the fused layer launch, timed with HIP events per replay on the
stream it is launched on -- and the CPU baseline (the reference's fp32
decode-row path restated in oracle/, timed on this host).

--profile ROLE runs only a calibration read of known size (the library's
speed-of-light read kernel) and one kind of launch -- the fused layer graph
(the timed region), or the scan, top-k or attention launches alone -- for
rocprofv3 kernel-trace and counter runs (--profile-main = --profile fused).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "dsa-multi-layer-indexer_amd"))
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
MALL_DEFEAT_BYTES = 768 << 20  # 3x the 256 MB Infinity Cache
TRAFFIC_FILE = REPO / "profiles" / "decode_layer_c3_hbm_traffic.md"
CONFIGS = {
    "c2": dict(lens=[32768], layers=2, indexer_every=1, desc="v32_ctx32768_b1_2layer_mli_graph"),
    "c3": dict(lens=[131072], layers=2, indexer_every=1, desc="v32_ctx131072_b1_2layer_mli_graph"),
    "c4": dict(lens=None, layers=2, indexer_every=1, desc="v32_varlen32_ctx16k-128k_2layer_mli_graph"),
    "c5": dict(lens=[196608], layers=61, indexer_every=4, desc="v32_ctx196608_b1_61layer_indexcache4_mli_graph"),
}


def scan_bytes(lens: list[int], hidx: int = 64) -> int:
    """Algorithmic HBM bytes of one scan launch: 128 B key + 4 B scale read
    and 4 B score written per token, the fp8 query, the weights and the
    page-table entries."""
    tok = sum(lens)
    pages = sum((n + 63) // 64 for n in lens)
    return 136 * tok + len(lens) * (hidx * 128 + hidx * 4) + 4 * pages


def attn_bytes(B: int, topk: int = 2048, H: int = 16) -> int:
    """Gathered latent rows + bf16 query + bf16 output per row."""
    return B * (topk * 656 + H * 576 * 2 + H * 512 * 2)


def time_graph(fn, iters: int, torch) -> float:
    """Average ms of fn() over iters, bracketed by synchronize."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / iters


def event_ms(fn, iters: int, torch) -> float:
    """Average per-launch device time of fn() with HIP events recorded on the
    stream fn launches on (torch's current stream), one event pair per launch."""
    pairs = []
    for _ in range(iters):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        pairs.append((a, b))
    torch.cuda.synchronize()
    return statistics.mean(a.elapsed_time(b) for a, b in pairs)


def graph_event_ms(fn, iters: int, torch) -> float:
    """Per-launch time of fn() from HIP events around one replay of a graph
    holding `iters` back-to-back launches (captured on torch's current
    stream, so the events bracket exactly those kernels)."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(iters):
                fn()
    torch.cuda.current_stream().wait_stream(s)
    g.replay()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def speed_of_light(lib, nbytes: int, torch, launches: int = 96) -> dict:
    """What one launch can reach on this part, timed like the scan (graph of
    back-to-back launches, HIP events): an empty launch, and a pure
    dependency-free read of `nbytes` per launch rotating over enough buffers
    (>= 768 MB) that every launch streams from HBM."""
    import ctypes

    dev = torch.device("cuda:0")
    nbuf = max(2, -(-MALL_DEFEAT_BYTES // nbytes))
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device=dev) for _ in range(nbuf)]
    sink = torch.zeros(16, dtype=torch.int32, device=dev)
    lib.dsa_internal_sol_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_void_p]
    lib.dsa_internal_sol_empty.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    st = {"i": 0}

    def read():
        lib.dsa_internal_sol_read(bufs[st["i"] % nbuf].data_ptr(), nbytes, sink.data_ptr(), 512,
                                  torch.cuda.current_stream().cuda_stream)
        st["i"] += 1

    def empty():
        lib.dsa_internal_sol_empty(sink.data_ptr(), 512, torch.cuda.current_stream().cuda_stream)
    read_ms = graph_event_ms(read, launches, torch)
    empty_ms = graph_event_ms(empty, launches, torch)
    del bufs
    return {"empty_launch_us": round(empty_ms * 1e3, 3), "read_us": round(read_ms * 1e3, 3),
            "read_bytes": nbytes, "read_GBps": round(nbytes / (read_ms * 1e-3) / 1e9, 1)}


def kernel_source_sha(root: Path = REPO) -> str:
    """sha256 (16 hex) over the HIP sources and the C header the library is
    built from, comments and whitespace left out: the kernels' memory
    traffic is a function of this code, not of its comments."""
    import hashlib
    import re

    h = hashlib.sha256()
    files = sorted((root / "dsa-multi-layer-indexer_amd" / "csrc").glob("*")) + [root / "include" / "dsa_mli.h"]
    for f in files:
        if f.suffix in (".hip", ".h"):
            code = re.sub(r"//[^\n]*|/\*.*?\*/", " ", f.read_text(), flags=re.S)
            h.update(f.name.encode())
            h.update(" ".join(code.split()).encode())
    return h.hexdigest()[:16]


def read_traffic():
    """HBM bytes per fused layer launch measured by the rocprofv3 counter runs
    (FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy) recorded in
    profiles/, with the kernel-source hash the counters were taken on.
    Returns (bytes or None, note): None when the summary is absent or was
    taken on other kernel sources (a stale figure is never reported)."""
    try:
        lines = TRAFFIC_FILE.read_text().splitlines()
    except OSError:
        return None, "no counter summary"
    vals = dict(l.split(":", 1) for l in lines if l.startswith(("traffic_bytes_per_launch:", "kernel_source_sha:")))
    sha = vals.get("kernel_source_sha", "").strip()
    if sha != kernel_source_sha():
        return None, f"counter summary taken on kernel sources {sha or '?'}, not these ({kernel_source_sha()})"
    try:
        return int(vals["traffic_bytes_per_launch"].strip()), f"rocprofv3 FETCH_SIZE+WRITE_SIZE, sources {sha}"
    except (KeyError, ValueError):
        return None, "no traffic line"


def cpu_baseline(ctx: int, budget_s: float = 15.0) -> dict:
    """The reference's fp32 decode-row path (oracle/cpu_reference_path.py) on
    this host's cores, bounded to about budget_s seconds."""
    import torch

    from oracle.cpu_reference_path import decode_layer_fp32, make_inputs

    inp = make_inputs(ctx, seed=0)
    decode_layer_fp32(*inp, topk=2048)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        decode_layer_fp32(*inp, topk=2048)
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    return {"value": statistics.median(times) * 1e6, "unit": "us/layer",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(times)} fp32 decode layers (indexer_logits -> select_topk -> "
                      f"masked _attend) at ctx {ctx}, b=1, median"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--nsplit", type=int, default=0,
                    help="attention splits per (row, head group); 0 = the library's choice")
    ap.add_argument("--scores", choices=["uniform", "window"], default="uniform",
                    help="window: the keys of a 3000-token window of each row (from position len/3) "
                         "score 50x the rest, so each row's top-2048 is packed in a few positions "
                         "(a recent-token-heavy selection)")
    ap.add_argument("--max-sets", type=int, default=64,
                    help="cap on the rotated layer sets (1: no Infinity-Cache defeat)")
    ap.add_argument("--profile", choices=["fused", "scan", "topk", "attn", "two_stream"], default=None,
                    help="only the calibration read and one kind of launch (profiler runs)")
    ap.add_argument("--profile-main", action="store_true", help="= --profile fused")
    ap.add_argument("--graph-packet-capture", action="store_true",
                    help="keep the HIP runtime's default graph launch mode (captured AQL packets), "
                         "which adds ~3.5 us to every replay")
    args = ap.parse_args()
    if args.profile_main:
        args.profile = "fused"
    # The HIP runtime replays a graph either from AQL packets it captured at
    # instantiation (its default) or by launching the graph's nodes on the
    # stream.  On this stack the first costs ~4.7 us per replay more than
    # eager launches, the second ~1.2 us; the kernels and their order are the
    # same.  Read once at runtime start-up, so it is set before torch loads.
    if not args.graph_packet_capture:
        os.environ.setdefault("DEBUG_CLR_GRAPH_PACKET_CAPTURE", "0")
    packet_capture = os.environ.get("DEBUG_CLR_GRAPH_PACKET_CAPTURE", "1") != "0"
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (one TP-8 share of heads); "
                                   "multi-GPU runs are not part of it", "n_gpus": args.gpus}))
        return 2

    import torch

    from lagged_indexer_dsa_amd import _lib, ops
    from lagged_indexer_dsa_amd import synthetic as S
    from lagged_indexer_dsa_amd.decode import MLISchedule

    dev = torch.device("cuda:0")
    cfg = CONFIGS[args.config]
    lens = cfg["lens"]
    if lens is None:
        g = torch.Generator().manual_seed(4000)
        lens = torch.randint(16384, 131073, (32,), generator=g).tolist()
    B = len(lens)
    n_layers = cfg["layers"]
    pt, num_pages = S.make_page_table(lens, seed=1000, device=dev)
    # The scanned index cache and gathered rows of one step (about 37 MB at
    # C3) would stay in the 256 MB Infinity Cache across replays; a real
    # model's layers never revisit theirs within a step.  Replays therefore
    # rotate over enough independent layer sets that each one streams its
    # inputs from HBM (every set is touched once per `n_sets` replays).
    step_bytes = (sum(1 for i in range(n_layers) if i % cfg["indexer_every"] == 0) * scan_bytes(lens)
                  + n_layers * attn_bytes(B))
    n_sets = max(1, min(args.max_sets, -(-MALL_DEFEAT_BYTES // step_bytes)))
    sets = []
    for k in range(n_sets):
        layers = [S.make_decode_layer(lens, seed=1000 * 3 + 100 * k + i, device=dev, page_table=pt,
                                      num_pages=num_pages, indexer=(i % cfg["indexer_every"] == 0),
                                      nsplit=args.nsplit)
                  for i in range(n_layers)]
        sets.append(layers)
    if args.scores == "window":
        # scale the key scales of each row's window: every score there is
        # 50x (the scores are linear in the key scale)
        pos = torch.cat([torch.arange(n // 3, min(n, n // 3 + 3000)) for n in lens])
        row = torch.cat([torch.full((min(n, n // 3 + 3000) - n // 3,), r) for r, n in enumerate(lens)])
        ptc = pt.cpu()
        pg = ptc[row, pos // 64].long().to(dev)
        slot = (pos % 64).to(dev)
        for ls in sets:
            for L in ls:
                if L.has_indexer:
                    sc = L.index_k.view(num_pages, -1)[:, 8192:].view(torch.float32)
                    sc[pg, slot] *= 50.0
    layers = sets[0]
    first = S.random_selection(lens, 2048, pt, seed=7, device=dev)
    torch.cuda.synchronize()

    fulls = [MLISchedule(ls, first) for ls in sets]
    full = fulls[0]
    attn_onlys = [MLISchedule(ls, first, indexer=False, attend_all_first=True) for ls in sets]
    idx_onlys = [MLISchedule(ls, first, attention=False) for ls in sets]
    scheds = fulls + attn_onlys + idx_onlys
    for s in scheds:
        s.capture()
    # set-up, not warm-up steps: each graph's first launch (the runtime
    # uploads the executable graph then) and first touch of its set's
    # buffers, so that a short run (--steps 20 --warmup 5 touches only a few
    # of the rotated sets before timing) measures the steady state
    if not args.profile:  # (profiler runs keep their kernel counts to the timed launches)
        for s in scheds:
            s.replay()
        torch.cuda.synchronize()

    def rotated(group):
        state = {"i": 0}

        def fn():
            group[state["i"] % len(group)].replay()
            state["i"] += 1
        return fn

    L0s = [ls[0] for ls in sets]

    def rot_layers(make):
        fns = [make(L) for L in L0s]
        state = {"i": 0}

        def fn():
            fns[state["i"] % len(fns)]()
            state["i"] += 1
        return fn
    scan = rot_layers(lambda L: lambda: ops.indexer_scan(L.q_fp8, L.w, L.index_k, L.page_table,
                                                         L.seq_lens, L.slab_stride, out=L.scores))
    topk_fn = rot_layers(lambda L: lambda: ops.topk(L.scores, L.seq_lens, 2048, page_table=L.page_table,
                                                    out=L.next_idx, scratch=L.topk_scratch))
    attn_fn = rot_layers(lambda L: lambda: ops.sparse_mla_decode(L.q_bf16, L.kv_pool, first, nsplit=L.nsplit,
                                                                 workspace=L.workspace, out=L.out))

    if args.profile:
        # calibration for the HBM byte counters: the speed-of-light read
        # kernel over buffers of the scan's size (its bytes are known)
        sol = speed_of_light(_lib.load(), scan_bytes(lens), torch, launches=20)
        if args.profile == "two_stream":
            # the second-stream design: attention launches on one stream,
            # scan launches on another, no ordering between the two; the
            # kernel trace shows whether their executions overlap
            sa, sb2 = torch.cuda.Stream(), torch.cuda.Stream()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(max(20, args.steps)):
                with torch.cuda.stream(sa):
                    attn_fn()
                with torch.cuda.stream(sb2):
                    scan()
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3 / max(20, args.steps)

            # the same pair as graphs (no host launch cost): two branches
            # forked from one stream and joined, against one stream
            def pair_graph(two: bool):
                g = torch.cuda.CUDAGraph()
                cap = torch.cuda.Stream()
                cap.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(cap):
                    with torch.cuda.graph(g, stream=cap):
                        for _ in range(20):
                            if two:
                                sa.wait_stream(cap)
                                sb2.wait_stream(cap)
                                with torch.cuda.stream(sa):
                                    attn_fn()
                                with torch.cuda.stream(sb2):
                                    scan()
                                cap.wait_stream(sa)
                                cap.wait_stream(sb2)
                            else:
                                attn_fn()
                                scan()
                torch.cuda.current_stream().wait_stream(cap)
                return g

            def replay_ms(g):
                g.replay()
                torch.cuda.synchronize()
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                for _ in range(5):
                    g.replay()
                b.record()
                torch.cuda.synchronize()
                return a.elapsed_time(b) / (5 * 20)
            g2, g1 = pair_graph(True), pair_graph(False)
            two_ms, one_ms = replay_ms(g2), replay_ms(g1)
            for s in scheds:
                s.close()
            print(json.dumps({"profile": "two_stream", "eager_ms_per_pair": round(ms, 5),
                              "graph_two_branches_ms_per_pair": round(two_ms, 5),
                              "graph_one_stream_ms_per_pair": round(one_ms, 5)}), flush=True)
            return 0
        if args.profile != "fused":
            fn = {"scan": scan, "topk": topk_fn, "attn": attn_fn}[args.profile]
            for _ in range(args.warmup):
                fn()
            torch.cuda.synchronize()
            ms = graph_event_ms(fn, max(20, args.steps), torch)
            for s in scheds:
                s.close()
            print(json.dumps({"profile": args.profile, "sets": n_sets, "launch_us": round(ms * 1e3, 3),
                              "calibration": sol}), flush=True)
            return 0

    _lib.sync_timeouts(reset=True)
    for i in range(args.warmup):
        fulls[i % n_sets].replay()
    # ---- timed region: exactly `steps` graph replays, bracketed by one HIP
    # event pair on the stream the graphs are launched on ----
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for i in range(args.steps):
        fulls[i % n_sets].replay()
    ev1.record()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    # the fused launches hand data between workgroups through bounded waits;
    # an expired wait means wrong (and fast) results: refuse to report them
    n_timeouts = _lib.sync_timeouts()
    if n_timeouts:
        print(json.dumps({"error": f"{n_timeouts} in-launch group waits expired in the timed region; "
                                   "results invalid", "config": cfg["desc"]}), flush=True)
        return 3
    # every replay is n_layers launches of the one kernel; the figure includes
    # the launch-to-launch gaps, so it bounds the kernel's duration from above
    launch_ms = ev0.elapsed_time(ev1) / (args.steps * n_layers)
    # per launch, averaged over the step's layers (IndexCache layers run no scan)
    n_idx = sum(1 for i in range(n_layers) if i % cfg["indexer_every"] == 0)
    lb = (n_idx * scan_bytes(lens) + n_layers * attn_bytes(B)) // n_layers
    if args.profile:
        for s in scheds:
            s.close()
        print(json.dumps({"profile": "fused", "sets": n_sets, "us_per_layer": round(ms_step * 1e3 / n_layers, 3),
                          "launch_us": round(launch_ms * 1e3, 3), "layer_bytes": lb,
                          "calibration": sol}), flush=True)
        return 0

    # graph steps of the three kinds (a fixed count, after a warm-up of each
    # kind, so the figure does not depend on --steps)
    reps = 100
    for grp in (attn_onlys, idx_onlys, fulls):
        time_graph(rotated(grp), 2 * n_sets, torch)
    t_attn = time_graph(rotated(attn_onlys), reps, torch)
    t_idx = time_graph(rotated(idx_onlys), reps, torch)
    t_full = time_graph(rotated(fulls), reps, torch)
    hidden = 1.0 - (t_full - t_attn) / t_idx if t_idx > 0 else None
    # the same from the launches' device time (a graph of back-to-back
    # launches of one kind, HIP events around it): no step replay overhead
    import ctypes as _ct

    def layer_launch(kind):
        argsets = [ls[0].args(first, indexer=(kind != "attn"), attention=(kind != "idx")) for ls in sets]
        st = {"i": 0}

        def fn():
            _lib.call("dsa_decode_layer", _ct.byref(argsets[st["i"] % len(argsets)]),
                      torch.cuda.current_stream().cuda_stream)
            st["i"] += 1
        return fn
    nk = max(48, 2 * n_sets)
    k_full = graph_event_ms(layer_launch("full"), nk, torch)
    k_attn = graph_event_ms(layer_launch("attn"), nk, torch)
    k_idx = graph_event_ms(layer_launch("idx"), nk, torch)
    hidden_k = 1.0 - (k_full - k_attn) / k_idx if k_idx > 0 else None
    # the same schedule without a graph, over the same rotated sets
    eager_state = {"i": 0}

    def eager_rotated():
        fulls[eager_state["i"] % len(fulls)].run_eager()
        eager_state["i"] += 1
    t_eager = time_graph(eager_rotated, reps, torch)
    # and layer by layer (one set, cache-warm)

    def serial():
        att = first
        for L in layers:
            L.run(attend_idx=att)
            if L.has_indexer:
                att = L.next_idx
    t_serial = time_graph(serial, reps, torch)

    # ---- the standalone ops (scan-only launches, the top-k (position order: one select launch), the
    # attention alone), each rotating over the sets' first layers ----
    for _ in range(10):
        scan()
    n_graph = max(50, 2 * n_sets)
    scan_ms = graph_event_ms(scan, n_graph, torch)
    scan_ms_pairs = event_ms(scan, 100, torch)
    sb = scan_bytes(lens)
    scan_gbs = sb / (scan_ms * 1e-3) / 1e9
    topk_ms = graph_event_ms(topk_fn, n_graph, torch)
    attn_ms = graph_event_ms(attn_fn, n_graph, torch)
    ab = attn_bytes(B)
    # decode-step operand preparation for one layer: quantize the indexer
    # query, append each row's newest key and latent row (the token at
    # seq_len - 1, rewritten in place)
    Lp = L0s[0]
    gq = torch.Generator(device=dev).manual_seed(11)
    q_idx = torch.randn(B, 64, 128, generator=gq, device=dev).to(torch.bfloat16)
    w_idx = torch.randn(B, 64, generator=gq, device=dev) / 8
    new_k = torch.randn(B, 128, generator=gq, device=dev).to(torch.bfloat16)
    new_lat = torch.randn(B, 576, generator=gq, device=dev).to(torch.bfloat16)
    rows_i = torch.arange(B, dtype=torch.int32, device=dev)
    pos_i = (Lp.seq_lens - 1).to(torch.int32)
    slot_i = torch.gather(Lp.page_table.long(), 1, (pos_i.long() // 64)[:, None])[:, 0] * 64 + pos_i.long() % 64
    slot_i = slot_i.to(torch.int32)
    q8_buf = torch.empty(B, 64, 128, dtype=torch.uint8, device=dev)
    w8_buf = torch.empty(B, 64, dtype=torch.float32, device=dev)

    def prep():
        ops.quantize_index_query(q_idx, w_idx, out_q=q8_buf, out_w=w8_buf)
        ops.append_index_keys(Lp.index_k, Lp.page_table, rows_i, pos_i, new_k)
        ops.append_latent_rows(Lp.kv_pool, slot_i, new_lat)
    prep_ms = graph_event_ms(prep, 50, torch)

    sol = speed_of_light(_lib.load(), sb, torch)
    traffic, traffic_note = read_traffic()
    us_layer = ms_step * 1e3 / n_layers
    layer_gbs = lb / (launch_ms * 1e-3) / 1e9
    res = {
        "metric": ("\u00b5s per DSA decode layer at 128K ctx (b=1, 16 heads); indexer-scan HBM GB/s"
                   if args.config == "c3" else f"\u00b5s per DSA decode layer ({args.config})"),
        "value": round(us_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3-indexer/fp8-kv-bf16-mla/fp32-accum",
        "data": "synthetic N(0,1), seeded, fp8-quantised paged caches (64-token pages, random page table)",
        "config": {"workload": cfg["desc"], "batch": B, "ctx": lens if B <= 4 else
                   {"min": min(lens), "max": max(lens), "sum": sum(lens)},
                   "layers_per_step": n_layers, "index_heads": 64, "attn_heads": 16,
                   "topk": 2048, "page_tokens": 64,
                   "schedule": "MLI lag, one fused launch per layer, 1 hipGraph",
                   "hip_graph_packet_capture": packet_capture,
                   "rotated_sets": n_sets, "bytes_per_step": step_bytes, "scores": args.scores},
        "tokens_per_s": round(B / (us_layer * 1e-6), 1),
        "indexer_scan_GBps": round(scan_gbs, 1),
        "layer_launch_us": round(launch_ms * 1e3, 3),
        "operand_prep_us": round(prep_ms * 1e3, 3),
        "kernel_us": {"indexer_scan": round(scan_ms * 1e3, 3), "topk": round(topk_ms * 1e3, 3),
                      "sparse_mla+combine": round(attn_ms * 1e3, 3),
                      "indexer_scan_event_pairs": round(scan_ms_pairs * 1e3, 3)},
        "attention_gather_GBps": round(ab / (attn_ms * 1e-3) / 1e9, 1),
        # the scan against what one launch of its bytes can reach here
        "speed_of_light": dict(sol, indexer_scan_frac=round(sol["read_us"] / (scan_ms * 1e3), 4)),
        "mli": {"graph_ms": round(t_full, 5), "eager_ms": round(t_eager, 5),
                "serial_ms": round(t_attn + t_idx, 5),
                "eager_layer_calls_ms": round(t_serial, 5), "attn_only_ms": round(t_attn, 5),
                "indexer_only_ms": round(t_idx, 5),
                "hidden_fraction": None if hidden is None else round(hidden, 4),
                # the largest hidden fraction possible: the indexer can only
                # hide under the attention's own time, so with the attention
                # the shorter of the two the bound is t_attn / t_idx
                "hidden_bound": None if t_idx <= 0 else round(min(1.0, t_attn / t_idx), 4),
                # the other side: the share of the attention's time the step
                # does not add on top of the indexer alone
                "attention_hidden_fraction": None if t_attn <= 0 else round(1.0 - (t_full - t_idx) / t_attn, 4),
                # per launch (device time of back-to-back launches of one
                # kind): fused layer, attention alone, indexer (scan + select)
                # alone, and the hidden fraction they give
                "kernel_us": {"fused": round(k_full * 1e3, 3), "attention_only": round(k_attn * 1e3, 3),
                              "indexer_only": round(k_idx * 1e3, 3)},
                "hidden_fraction_kernels": None if hidden_k is None else round(hidden_k, 4),
                "hidden_bound_kernels": None if k_idx <= 0 else round(min(1.0, k_attn / k_idx), 4)},
        "roofline": {"bound": "hbm", "achieved": round(layer_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic if args.config == "c3" and args.scores == "uniform" else None,
                     "traffic_source": traffic_note if args.config == "c3" and args.scores == "uniform"
                     else "the counter summary covers the C3 launch only",
                     "kernel": "decode_main_kernel (fused layer launch)" if B < 8 else
                     "flat_scan_kernel (scan, attention riding) + decode_main_kernel (select): the layer's launches",
                     "algorithmic_bytes": lb, "launch_us": round(launch_ms * 1e3, 3)},
    }
    n_timeouts = _lib.sync_timeouts()
    if n_timeouts:
        print(json.dumps({"error": f"{n_timeouts} in-launch group waits expired outside the timed region"}),
              flush=True)
        return 3
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(131072 if args.config == "c3" else 8192, args.cpu_budget)
        if args.config == "c3":  # and at C1's context (8192 tokens, the reference's CPU-runnable case)
            res["cpu_baseline_c1"] = cpu_baseline(8192, min(5.0, args.cpu_budget))
    for s in scheds:
        s.close()
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
