"""Benchmark of the MI355X quantized decode hot path (one JSON line on stdout).

Metric: INT4 GEMV HBM GB/s (% of peak) at Qwen3-1.7B shapes, batch 1.

Workload (the INT4 half of the batch-1 GEMV sweep at its
real model scale): one step = the INT4 group-128 dequant-GEMV of every linear
weight of a 28-layer Qwen3-1.7B-shaped decoder -- per layer q [2048x2048],
k/v [1024x2048], o [2048x2048], gate/up [6144x2048], down [2048x6144] --
196 GEMVs, 750,862,336 algorithmic bytes (packed weights + fp32 scales +
fp16 x + fp16 y), each weight resident in HBM and touched once per step
(751 MB > the 256 MB Infinity Cache, so reads come from HBM). The 196
independent GEMVs run as ONE grouped launch per step (4 shape classes).
value = algorithmic bytes / step time, timed over --steps steps between two
device synchronisations, after --ramp-ms (default 250) of untimed steps and
--warmup steps (the loaded steady state: the first hundred or so launches
after set-up run up to ~10% slower).

The last stdout line is the compact result: the headline fields, config,
roofline (the dominant -- and only -- launch of a step; its average duration
from two HIP events on the launching stream around the timed steps themselves,
so it cannot exceed ms_per_step; `traffic` is the HBM bytes per launch from the
FETCH_SIZE / WRITE_SIZE counter summary committed under profiles/, null when
absent), decode_tok_s (config 5 per mode) and cpu_baseline. Everything else is
one 'bench-detail: {...}' line on stderr (and --detail-json PATH):
  batched_per_class  the same GEMVs as one launch per shape class, per class;
  int8_batched_per_class  the INT8 g128 GEMVs of the same shapes, one batched launch per class;
  copy_reference  a plain device-to-device copy of 512 MiB (the calibration
                  kernel of the counter runs, and the box's streaming rate), and
                  by_size: the same copy of one gate/up GEMV's bytes, of 64 MB and of a step;
  decode_chain    the 112 dependent launches of one decode step, graph-replayed;
  per_shape_cold  per-shape INT4 / INT8 single-launch times on cold copies;
  topk_us_I6144   top-k latency at I=6144;
  kernels         every other hot-path kernel at its BASELINE shape on cold copies:
                  bytes, us per launch, GB/s, fraction of the HBM peak;
  dip_mlp_layer   BASELINE configs 3-4: one layer's dense / DIP (k/I 0.125, 0.25, 0.5) / cache-aware
                  DIP MLP, graph-replayed over 28 distinct layers;
  decode          BASELINE config 5: greedy decode tok/s of the random-init 28-layer Qwen3-1.7B
                  shape, dense vs DIP vs cache-aware DIP at k/I = 0.5 (64-token prompt, 128 tokens);
  cpu_baseline    the reference's CPU GEMV path (dequantize + fp32 torch.mv) on layer 0's GEMVs,
                  at the job's host cores and one thread, and the other operators' CPU oracles.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--ramp-ms MS]
       python bench.py --traffic-set   (only the launches of the HBM counter passes whose summaries are
                                        committed under profiles/; prints their algorithmic bytes)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for p in (str(REPO / "sparse-offload-infer_amd"), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
LAYERS = 28
H, I, NQ, NKV, HD, GS = 2048, 6144, 16, 8, 128, 128
# (name, N, K) per layer, in decode order
LAYER_SHAPES = [("q", NQ * HD, H), ("k", NKV * HD, H), ("v", NKV * HD, H), ("o", H, NQ * HD),
                ("gate", I, H), ("up", I, H), ("down", H, I)]
METRIC = "INT4 GEMV HBM GB/s (% of peak); DIP decode tok/s, Qwen3-1.7B shape, bs=1"


def log(msg: str) -> None:
    """Progress line on stderr (stdout carries only the JSON result)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def int4_bytes(N: int, K: int, gs: int = GS) -> int:
    """Algorithmic bytes of one INT4 GEMV: packed weights + fp32 scales + fp16 x + fp16 y."""
    return N * ((K + 7) // 8) * 4 + N * ((K + gs - 1) // gs) * 4 + 2 * K + 2 * N


def int8_bytes(N: int, K: int, gs: int = GS) -> int:
    return N * K + N * ((K + gs - 1) // gs) * 4 + 2 * K + 2 * N


def make_int4(N, K, gen, device):
    import torch

    from soinfer.quant import formats, pack

    w = torch.randn(N, K, generator=gen, device=device) * 0.02
    qt = formats.quantize(w, formats.QuantConfig(bits=4, granularity="group", group_size=GS))
    Wq, _ = pack.pack_int4(qt.qweight)
    return Wq.contiguous(), qt.scale.contiguous()


def make_int8(N, K, gen, device):
    import torch

    from soinfer.quant import formats

    w = torch.randn(N, K, generator=gen, device=device) * 0.02
    qt = formats.quantize(w, formats.QuantConfig(bits=8, granularity="group", group_size=GS))
    return qt.qweight.contiguous(), qt.scale.contiguous()


def time_back_to_back(fn, launches: int = 30):
    """Average duration of `launches` back-to-back launches: two HIP events on the launching (current) stream."""
    import torch

    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(launches):
        fn()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) * 1e3 / launches  # microseconds


def time_graph_per_launch(fn, args_list, reps: int = 5):
    """Per-launch time of back-to-back launches (each on its own cold copy) captured in one HIP graph."""
    import torch

    for a in args_list[:4]:
        fn(*a)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for a in args_list:
            fn(*a)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / (reps * len(args_list)) * 1e6
    # per-replay spread (HIP events around each replay)
    per = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        per.append(a.elapsed_time(b) * 1e3 / len(args_list))
    per.sort()
    return {"mean_us": us, "median_us": per[len(per) // 2], "p90_us": per[min(len(per) - 1, int(0.9 * len(per)))]}


TRAFFIC_FILE = REPO / "profiles" / "gemv_int4_grouped_qwen3_1p7b_step_traffic.md"


def read_traffic(path: Path = TRAFFIC_FILE):
    """HBM bytes per dominant launch from the committed counter summary (line `traffic_bytes_per_launch: N`)."""
    import re

    try:
        m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)\s*$", path.read_text(), re.M)
    except OSError:
        return None
    return int(m.group(1)) if m else None


def copy_reference(nbytes: int = 512 << 20, reps: int = 10):
    """A plain device-to-device copy of `nbytes` (torch's copy kernel): read + write bytes / kernel time."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_(0, 256)
    dst = torch.empty_like(src)
    dst.copy_(src)
    us = time_back_to_back(lambda: dst.copy_(src), launches=reps)
    del src, dst
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us": round(us, 2),
            "GBps": round(2 * nbytes / (us * 1e-6) / 1e9, 1)}


def cold_copies(nbytes: int, target: int = 600 << 20) -> int:
    return max(8, -(-target // nbytes))


def bench_shapes(ops, dev, gen):
    """Per-shape INT4 / INT8 kernel time on rotating cold copies."""
    import torch

    out = {}
    shapes = [("gate_up_6144x2048", 6144, 2048), ("down_2048x6144", 2048, 6144), ("q_o_2048x2048", 2048, 2048),
              ("k_v_1024x2048", 1024, 2048)]
    for name, N, K in shapes:
        b4 = int4_bytes(N, K)
        n = cold_copies(b4)
        base_W, base_s = make_int4(N, K, gen, dev)
        Ws = [base_W.clone() for _ in range(n)]
        Ss = [base_s.clone() for _ in range(n)]
        x = torch.randn(K, generator=gen, device=dev).half()
        args = [(Ws[i], Ss[i], x, K, GS) for i in range(n)]
        t = time_graph_per_launch(ops.gemv_w4a16_group_lop3, args, reps=10)
        # warm: the same copy every launch (6.7 MB stays in the 256 MB memory-side cache), labelled separately
        tw = time_graph_per_launch(ops.gemv_w4a16_group_lop3, [args[0]] * n, reps=10)
        out[name] = {"int4_bytes": b4, "int4_us": round(t["mean_us"], 3), "int4_p90_us": round(t["p90_us"], 3),
                     "int4_GBps": round(b4 / t["mean_us"] / 1e3, 1),
                     "int4_frac_of_hbm": round(b4 / (t["mean_us"] * 1e-6) / HBM_PEAK, 4),
                     "int4_warm_us": round(tw["mean_us"], 3)}
        del Ws, Ss, args
        b8 = int8_bytes(N, K)
        n8 = cold_copies(b8)
        q8, s8 = make_int8(N, K, gen, dev)
        Q8 = [q8.clone() for _ in range(n8)]
        S8 = [s8.clone() for _ in range(n8)]
        args8 = [(Q8[i], S8[i], x, GS) for i in range(n8)]
        t8 = time_graph_per_launch(ops.gemv_w8a16, args8, reps=10)
        out[name].update({"int8_bytes": b8, "int8_us": round(t8["mean_us"], 3), "int8_p90_us": round(t8["p90_us"], 3),
                          "int8_GBps": round(b8 / t8["mean_us"] / 1e3, 1),
                          "int8_frac_of_hbm": round(b8 / (t8["mean_us"] * 1e-6) / HBM_PEAK, 4)})
        del Q8, S8, args8
        torch.cuda.empty_cache()
    return out


def bench_topk(ops, dev, gen):
    import torch

    res = {}
    gate = (torch.randn(6144, generator=gen, device=dev) * 0.9).half().float().abs().contiguous()
    for frac in (0.125, 0.25, 0.5):
        k = int(6144 * frac)
        t = time_graph_per_launch(lambda v, kk: ops.topk_threshold_select(v, kk), [(gate, k)] * 64)
        res[f"k_{k}"] = round(t["mean_us"], 3)
    return res


def bench_decode_chain(ops, layers, step_bytes):
    """One decode step as 112 dependent launches (qkv and gate|up rows concatenated), replayed as a HIP graph."""
    import torch

    # ---- decode chain: per layer qkv (concatenated rows), o, gate|up (concatenated), down; dependent order ----
    chain = []
    for l in range(LAYERS):
        m = layers[l]
        qkv_W = torch.cat([m["q"][0], m["k"][0], m["v"][0]]).contiguous()
        qkv_s = torch.cat([m["q"][1], m["k"][1], m["v"][1]]).contiguous()
        gu_W = torch.cat([m["gate"][0], m["up"][0]]).contiguous()
        gu_s = torch.cat([m["gate"][1], m["up"][1]]).contiguous()
        chain.append([(qkv_W, qkv_s, m["q"][2], H), (m["o"][0], m["o"][1], m["o"][2], H),
                      (gu_W, gu_s, m["gate"][2], H), (m["down"][0], m["down"][1], m["down"][2], I)])

    def chain_step():
        for launches in chain:
            for W, s, x, K in launches:
                ops.gemv_w4a16_group_lop3(W, s, x, K, GS)

    chain_step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain_step()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    creps = 20
    for _ in range(creps):
        graph.replay()
    torch.cuda.synchronize()
    chain_s = (time.perf_counter() - t0) / creps
    decode_chain = {"ms_per_step": round(chain_s * 1e3, 4), "GBps": round(step_bytes / chain_s / 1e9, 1),
                    "frac_of_hbm": round(step_bytes / chain_s / HBM_PEAK, 4), "launches_per_step": 4 * LAYERS,
                    "note": "one launch per dependent GEMV of a decode step (qkv and gate|up rows concatenated), "
                            "HIP-graph replay"}
    del chain, graph
    return decode_chain

def mlp_bytes(L, I: int, H: int, k=None, dense_up: bool = False, gated: bool = False) -> int:
    """Algorithmic bytes of one layer's MLP: dense reads gate|up and down; DIP reads gate, k rows of up and
    k rows of down^T (packed + fp32 scales), plus the fp16 vectors it reads and writes; the dense-up DIP schedule
    and the gated one with the ordered down read every gate|up row and every down^T value (their downs run over
    the transposed down_proj^T: unselected channels read and left out), and write then read gate and h of every
    channel; the gated schedule's row form (gated=True) reads every gate|up row and k rows of down^T, and writes
    gate and up of every channel, then reads the gates and the k selected up values."""
    row = L.gu_Wq.shape[1] + 4 * L.gu_scale.shape[1]
    if k is None:
        return 2 * I * row + L.down_Wq.numel() + 4 * L.down_scale.numel() + 2 * (H + 3 * I + H)
    row_t = L.down_T_Wq.shape[1] + 4 * L.down_T_scale.shape[1]
    if dense_up:
        return 2 * I * row + I * row_t + 2 * (H + 4 * I + H)
    if gated:
        return 2 * I * row + k * row_t + 2 * (H + 3 * I + k + H) + 4 * k
    return I * row + k * (row + row_t) + 2 * (H + I + 2 * k + H) + 4 * (I + k)


def graph_time_us(fn, reps: int = 10) -> float:
    """Average time of fn's launches captured once in a HIP graph and replayed `reps` times (two HIP events
    on the current stream around the replays)."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) * 1e3 / reps


def bench_dip_mlp(D, w, hot, dev):
    """BASELINE configs 3 and 4: one layer's DIP MLP (gate GEMV, top-k of |gate|, sparse up, SiLU gating, sparse
    down) at k/I in {0.125, 0.25, 0.5}, the dense MLP, and the cache-aware form at k/I = 0.5 with a 20% hot
    cache whose misses come from pinned host memory. Each figure is the time of the 28 layers' MLPs replayed
    from one graph, divided by 28 (28 distinct weight sets, 540 MB, so weights come from HBM)."""
    import torch

    c = w.config
    I, H = c.intermediate, c.hidden
    x = (torch.randn(H, generator=torch.Generator().manual_seed(1)).half()).to(dev)
    res = {}

    def run(eng):
        eng.h.copy_(x)
        torch.cuda.synchronize()
        return graph_time_us(lambda: [eng._mlp(l, L) for l, L in enumerate(w.layers)]) / c.layers

    eng = D.DecodeEngine(w, "dense", max_new_tokens=1)
    us = run(eng)
    nb = mlp_bytes(w.layers[0], I, H)
    import soinfer._C as C

    def dense_norm_mlp():
        """The engine's dense MLP: gate|up GEMV with the RMSNorm on load and the SwiGLU epilogue, then down."""
        for l, L in enumerate(w.layers):
            gW, gS = eng.gu_il[l]
            C.gemv_w4a16_rmsnorm_into(gW, gS, x, None, w.layers[0].post_norm, c.rms_eps, None, None, eng.mlp_h, H,
                                      c.group_size, True)
            C.gemv_w4a16_into(L.down_Wq, L.down_scale, eng.mlp_h, eng.down, I, c.group_size)
    us_n = graph_time_us(dense_norm_mlp) / c.layers
    res["dense"] = {"us": round(us_n, 2), "bytes": nb, "GBps": round(nb / us_n / 1e3, 1),
                    "schedule": "gate|up GEMV with RMSNorm on load and SwiGLU epilogue, down GEMV (2 launches)",
                    "unfused_us": round(us, 2)}
    del eng

    def fused_dip(eng):
        """The engine's fused DIP MLP schedule without the RMSNorm prologue: gate GEMV, top-k of |gate|, up GEMV
        over the selected rows with the SiLU gating in its epilogue, sparse down (4 launches)."""
        gs = c.group_size

        def mlp():
            for L in w.layers:
                gW, gS = L.gate(I)
                uW, uS = L.up(I)
                gate = eng.gu[:I]
                C.gemv_w4a16_into(gW, gS, eng.h, gate, H, gs)
                C.topk_threshold_select_f16abs_into(gate, eng.k, eng.idx, eng.cnt)
                C.gemv_w4a16_indexed_silu_into(uW, uS, eng.idx, eng.h, gate, eng.h_sel, H, gs)
                C.gemv_w4a16_indexed_accumulate_into(L.down_T_Wq, L.down_T_scale, eng.idx, eng.h_sel, eng.down, H, gs,
                                                     eng.sd_ws)
        eng.h.copy_(x)
        torch.cuda.synchronize()
        return graph_time_us(mlp) / c.layers

    nw = w.layers[0].post_norm
    eps = c.rms_eps

    def norm_mlp(eng):
        """The engine's DIP MLP schedule with its RMSNorm on load (x -> rmsnorm -> MLP): the norm-fused gate GEMV,
        top-k, the up GEMV with the SiLU epilogue, the sparse down (4 launches)."""
        gs = c.group_size

        def mlp():
            for L in w.layers:
                gW, gS = L.gate(I)
                uW, uS = L.up(I)
                gate = eng.gu[:I]
                C.gemv_w4a16_rmsnorm_into(gW, gS, x, None, nw, eps, None, eng.h, gate, H, gs, False)
                C.topk_threshold_select_f16abs_into(gate, eng.k, eng.idx, eng.cnt)
                C.gemv_w4a16_indexed_silu_into(uW, uS, eng.idx, eng.h, gate, eng.h_sel, H, gs)
                C.gemv_w4a16_indexed_accumulate_into(L.down_T_Wq, L.down_T_scale, eng.idx, eng.h_sel, eng.down, H,
                                                     gs, eng.sd_ws)
        torch.cuda.synchronize()
        return graph_time_us(mlp) / c.layers

    for frac in (0.125, 0.25, 0.5):
        k = int(I * frac)
        eng = D.DecodeEngine(w, "dip", dip_k=k, max_new_tokens=1)
        us = run(eng)
        nb = mlp_bytes(w.layers[0], I, H, k)
        y_unfused = eng.down.clone()
        us_f = fused_dip(eng)
        assert torch.equal(eng.down, y_unfused), "fused DIP MLP must equal the unfused one"
        us_4 = norm_mlp(eng)
        idx_dip, y_norm = eng.idx.clone(), eng.down.clone()  # layer 27's selection and y on rmsnorm(x)
        if frac == 0.5:
            y_dip = y_unfused
        del eng
        # gated schedule (the engine's dip_schedule="gated"): gate and up of every channel in one launch with the
        # RMSNorm on load, then the rule-A selection in each workgroup and the gated sparse down over the selected
        # down^T rows (2 launches); the same selection and y as the four-launch schedule, bit for bit
        eng = D.DecodeEngine(w, "dip", dip_k=k, max_new_tokens=1, dip_schedule="gated")

        def gated_mlp():
            for l, L in enumerate(w.layers):
                gW, gS = eng.gu_il[l]
                C.gemv_w4a16_rmsnorm_gate_up_into(gW, gS, x, None, nw, eps, None, eng.gu[:I], eng.gu[I:], H,
                                                  c.group_size)
                C.dip_select_gated_down_into(eng.gu[:I], eng.gu[I:], k, L.down_T_Wq, L.down_T_scale, eng.idx, eng.cnt,
                                             eng.down, H, c.group_size, eng.sd_ws)
        us_gr = graph_time_us(gated_mlp) / c.layers
        assert torch.equal(eng.idx, idx_dip) and torch.equal(eng.down, y_norm), \
            "the gated schedule must equal the four-launch schedule bit for bit"
        us_g = us_gr
        if eng.dip_gated_tr:  # the engine's form where the shape fits: the down over the transposed copy
            def gated_tr_mlp():
                for l, L in enumerate(w.layers):
                    gW, gS = eng.gu_il[l]
                    Wt, St = eng.down_tt[l]
                    C.gemv_w4a16_rmsnorm_swiglu_gate_into(gW, gS, x, None, nw, eps, None, eng.gu[:I], eng.gu[I:], H,
                                                          c.group_size)
                    C.dip_select_down_ordered_into(eng.gu[:I], eng.gu[I:], k, Wt, St, None, None, eng.down,
                                                   c.group_size)
            eng.down.zero_()
            us_g = graph_time_us(gated_tr_mlp) / c.layers  # as the engine runs it: no index outputs
            assert torch.equal(eng.down, y_norm), "the ordered down must equal the four-launch schedule bit for bit"
            Wt, St = eng.down_tt[c.layers - 1]
            C.dip_select_down_ordered_into(eng.gu[:I], eng.gu[I:], k, Wt, St, eng.idx, eng.cnt, eng.down,
                                           c.group_size)
            torch.cuda.synchronize()
            assert torch.equal(eng.idx, idx_dip) and torch.equal(eng.down, y_norm), \
                "the ordered down's selection must equal the four-launch schedule's"
        del eng
        # dense-up schedule (the engine's dip_dense_up): one launch computes gate and h = fp16(silu(gate) * up) of
        # every channel with the RMSNorm on load, a second the rule-A selection in each workgroup and the down
        # projection as a GEMV over the transposed down_proj^T (2 launches); the same selection, y within the
        # sparse accumulate's tolerance of the four-launch schedule's
        eng = D.DecodeEngine(w, "dip", dip_k=k, max_new_tokens=1, dip_dense_up=True)
        us_du_unfused = run(eng)  # gate GEMV, up GEMV, SiLU gating, selection + down (4 launches)
        gate, h_all = eng.gu[:I], eng.gu[I:]

        def dense_up_mlp():
            for l, L in enumerate(w.layers):
                gW, gS = eng.gu_il[l]
                Wt, St = eng.down_tt[l]
                C.gemv_w4a16_rmsnorm_swiglu_gate_into(gW, gS, x, None, nw, eps, None, gate, h_all, H, c.group_size)
                C.dip_select_dense_down_into(gate, h_all, k, Wt, St, None, None, eng.down, c.group_size)
        us_du = graph_time_us(dense_up_mlp) / c.layers
        # on layer 27's input x: the selection and y against the four-launch schedule's
        C.dip_select_dense_down_into(gate, h_all, k, *eng.down_tt[c.layers - 1], eng.idx, eng.cnt, eng.down,
                                     c.group_size)
        torch.cuda.synchronize()
        same_sel = bool(torch.equal(eng.idx, idx_dip))
        ydiff = (eng.down.float() - y_norm.float()).abs().max().item() / max(y_norm.float().abs().max().item(), 1e-30)
        res[f"dip_k{k}"] = {
            "k_over_I": frac, "us": round(us_du, 2), "bytes": mlp_bytes(w.layers[0], I, H, k, dense_up=True),
            "schedule": "gate|up GEMV with RMSNorm on load writing gate and h of every channel, then the rule-A "
                        "selection in every workgroup + the down as a GEMV over the transposed down_proj^T "
                        "(2 launches)",
            "selection_equal_indexed_up": same_sel, "y_normalized_diff_vs_indexed_up": round(ydiff, 6),
            "dense_up_unfused_us": round(us_du_unfused, 2),
            "indexed_up_us": round(us_4, 2), "indexed_up_bytes": nb,
            "indexed_up_schedule": "RMSNorm-fused gate GEMV, top-k, up GEMV over the selected rows with the SiLU "
                                   "epilogue, sparse down (4 launches)",
            "indexed_up_no_norm_us": round(us_f, 2), "indexed_up_unfused_us": round(us, 2),
            "gated_us": round(us_g, 2), "gated_row_form_us": round(us_gr, 2),
            "gated_bytes": mlp_bytes(w.layers[0], I, H, k, dense_up=True),
            "gated_row_form_bytes": mlp_bytes(w.layers[0], I, H, k, gated=True),
            "gated_schedule": "gate|up GEMV with RMSNorm on load writing gate and h of every channel, then the "
                              "rule-A selection in every workgroup + the down in the sparse accumulate's order over "
                              "the transposed down_proj^T (gated_row_form_us: gate and up stored, then the selection "
                              "+ gated sparse down over the selected down^T rows); 2 launches, equal to the "
                              "four-launch schedule bit for bit"}
        res[f"dip_k{k}"]["GBps"] = round(res[f"dip_k{k}"]["bytes"] / us_du / 1e3, 1)
        del eng
    k = I // 2
    notes = {"direct": "misses read in place from the pinned host arena by the up GEMV and the down accumulate "
                       "(no descriptors, gathers or staging)",
             "staged": "descriptors, then in-graph device gathers of the misses from pinned host memory into "
                       "staging, then the descriptor kernels (the reference's shape)"}
    for path in ("direct", "staged"):
        eng = D.DecodeEngine(w, "cached_dip", dip_k=k, hot_channels=hot, max_new_tokens=1, miss_path=path)
        us = run(eng)
        assert torch.equal(eng.down, y_dip), "cache-aware DIP must equal DIP bit for bit"
        import soinfer.ops as ops
        misses = int(ops.build_dip_descriptors(eng.idx, eng.caches[-1].slot_of)[2].item())
        key = f"cached_dip_k{k}" if path == "direct" else f"cached_dip_staged_k{k}"
        res[key] = {"k_over_I": 0.5, "hot_fraction": 0.2, "us": round(us, 2), "misses_last_layer": misses,
                    "bit_identical_to_dip": True,
                    "host_bytes_last_layer": misses * (w.layers[0].gu_Wq.shape[1] + w.layers[0].down_T_Wq.shape[1]),
                    "note": notes[path]}
        del eng
    return res


def bench_decode(D, w, hot, dev, n_prompt: int = 64, n_new: int = 128, hot_sweep=None):
    """greedy decoding of the random-init 28-layer Qwen3-1.7B-shaped INT4 decoder from a
    seeded 64-token prompt, 128 new tokens, dense vs DIP vs cache-aware DIP at k/I = 0.5 (20% hot cache,
    misses from pinned host memory). One HIP graph per token; decode_tok_s = new tokens / decode time,
    end_to_end_tok_s = new tokens / (prefill + decode) time (the reference's tokens/sec, bench_m7_pareto.py:87-90).
    hot_sweep: {mode name: per-layer hot sets} of further cache-aware DIP runs at other cache sizes."""
    import torch

    c = w.config
    I = c.intermediate
    prompt = torch.randint(0, c.vocab, (n_prompt,), generator=torch.Generator().manual_seed(7)).tolist()
    k = I // 2
    out, toks = {}, {}
    L0 = w.layers[0]
    attn_w = (L0.qkv_Wq.numel() + 4 * L0.qkv_scale.numel() + L0.o_Wq.numel() + 4 * L0.o_scale.numel())
    # "dip": the indexed schedule (gate GEMV, top-k, up GEMV over the selected rows, sparse down), the one the
    # cache-aware engines reproduce bit for bit; "dip_dense_up": the same selection with the up GEMV over every
    # row and the down as one dense GEMV over a transposed down_proj^T (y summed in another order)
    # "*_offload": copies on copy streams two layers ahead of the kernels; "*_offload_serial": each layer's copy
    # stream-ordered right before its kernels
    # "*_int4_head": the same schedule with the LM head quantized like the linears (INT4 g128 GEMV) instead of
    # the reference's fp16 head: config 5's "all weights INT4 g128"
    modes = ("dense", "dip", "dip_gated", "dip_dense_up", "cached_dip", "cached_dip_staged", "dense_int4_head",
             "dip_int4_head", "dip_gated_int4_head", "dip_dense_up_int4_head", "cached_dip_int4_head",
             "dense_offload", "dip_offload", "cached_dip_offload", "dense_offload_serial", "dip_offload_serial",
             "cached_dip_offload_serial")
    hot_sweep = hot_sweep or {}
    modes = modes + tuple(hot_sweep)
    no_hot = [[] for _ in range(c.layers)]
    Wq_h, S_h = D.quantize_lm_head(w)
    head_bytes = {False: w.lm_head.numel() * 2, True: Wq_h.numel() + 4 * S_h.numel()}
    for mode in modes:
        int4_head = mode.endswith("_int4_head")
        kind = mode.replace("_serial", "").replace("_int4_head", "")
        base = {"dip_dense_up": "dip", "dip_gated": "dip", "cached_dip_staged": "cached_dip",
                "dense_offload": "dense", "dip_offload": "cached_dip", "cached_dip_offload": "cached_dip"}.get(kind, kind)
        mode_hot = hot_sweep.get(mode, no_hot if kind == "dip_offload" else hot)
        if mode in hot_sweep:
            kind = base = "cached_dip"
        eng = D.DecodeEngine(w, base, dip_k=None if base == "dense" else k,
                             hot_channels=mode_hot if base == "cached_dip" else None,
                             max_new_tokens=n_new,
                             dip_schedule={"dip_dense_up": "dense_up", "dip_gated": "gated"}.get(kind),
                             miss_path="staged" if mode == "cached_dip_staged" else "direct",
                             offload=kind.endswith("_offload"), overlap_copy=not mode.endswith("_serial"),
                             int4_head=int4_head)
        eng.capture()
        eng.generate(prompt[:8], 8)  # warm up the graphs
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.reset()
        eng.prefill(prompt)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        eng.decode(n_new)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        toks[mode] = eng.log[:n_new].tolist()
        mlp = mlp_bytes(L0, I, c.hidden, None if base == "dense" else k, dense_up=kind in ("dip_dense_up", "dip_gated"))
        per_tok = c.layers * (attn_w + mlp) + head_bytes[int4_head]
        out[mode] = {"decode_tok_s": round(n_new / (t2 - t1), 1), "ms_per_token": round((t2 - t1) / n_new * 1e3, 4),
                     "end_to_end_tok_s": round(n_new / (t2 - t0), 1), "prefill_ms": round((t1 - t0) * 1e3, 2),
                     "weight_bytes_per_token": per_tok,
                     "weight_GBps": round(per_tok * n_new / (t2 - t1) / 1e9, 1)}
        if mode in hot_sweep:
            out[mode]["hot_fraction"] = round(len(mode_hot[0]) / I, 3)
        if eng.offload:
            out[mode]["streamed_bytes_per_token"] = eng.wstore.bytes_total
            out[mode]["streamed_GBps"] = round(eng.wstore.bytes_total * n_new / (t2 - t1) / 1e9, 1)
        del eng
        torch.cuda.empty_cache()
        log(f"decode {mode}: {out[mode]['decode_tok_s']} tok/s")
    out["cached_dip_tokens_equal_dip"] = all(toks["dip"] == toks[m] for m in ("cached_dip", "cached_dip_staged",
                                                                              *hot_sweep))
    out["dip_gated_tokens_equal_dip"] = toks["dip"] == toks["dip_gated"]
    assert out["dip_gated_tokens_equal_dip"], "the gated DIP schedule must generate the indexed schedule's tokens"
    assert toks["dip_int4_head"] == toks["dip_gated_int4_head"], "gated DIP must equal DIP (INT4 head)"
    out["cached_dip_int4_head_tokens_equal_dip_int4_head"] = toks["dip_int4_head"] == toks["cached_dip_int4_head"]
    assert out["cached_dip_int4_head_tokens_equal_dip_int4_head"], "cache-aware DIP must equal DIP (INT4 head)"
    assert out["cached_dip_tokens_equal_dip"], "cache-aware DIP must generate the same tokens as DIP"
    for a, b in (("dense_offload", "dense"), ("dip_offload", "dip"), ("cached_dip_offload", "dip"),
                 ("dense_offload_serial", "dense"), ("dip_offload_serial", "dip"),
                 ("cached_dip_offload_serial", "dip")):
        assert toks[a] == toks[b], f"{a} must generate the same tokens as {b}"
    out["offload_tokens_equal_resident"] = True
    out["offload_note"] = ("*_offload: every layer's dense weights (q|k|v, o, gate|up and down for dense, gate for "
                           "DIP) streamed from a pinned host arena into one of two device slots by one hipMemcpyAsync "
                           "per layer on a copy stream, two layers ahead of the kernels (read-done fences; the first "
                           "two layers' copies overlap the LM head): the reference's streamed configuration with "
                           "WeightPipeline's prefetch; *_offload_serial: each copy stream-ordered right before its "
                           "layer. DIP reads its selected up / down^T rows from the host arena in place (dip_offload: "
                           "no cache, cached_dip_offload: 20% hot cache in HBM)")
    out["cached_dip"]["miss_path"] = "direct: misses read in place from the pinned host arena inside the GEMVs"
    out["cached_dip_staged"]["miss_path"] = "staged: device gathers of the misses into staging, then descriptors"
    out["dip"]["schedule"] = ("RMSNorm-fused gate GEMV, top-k, up GEMV with SiLU epilogue, sparse "
                              "down (4 launches per MLP); cached_dip equals it bit for bit")
    out["dip_gated"]["schedule"] = ("gate|up GEMV with RMSNorm on load writing gate and up of every channel, then the "
                                    "rule-A selection in every workgroup + the gated sparse down over the selected "
                                    "down^T rows (2 launches per MLP); dip's tokens and hidden states bit for bit")
    out["dip_dense_up_tokens_equal_dip"] = toks["dip"] == toks["dip_dense_up"]
    out["dip_dense_up"]["schedule"] = ("gate|up GEMV with RMSNorm on load writing gate and h of every channel, then the "
                              "rule-A selection in every workgroup + the down as a GEMV over the transposed "
                              "down_proj^T (2 launches per MLP); the selections of dip, y summed in "
                              "another order")
    out["config"] = {"prompt_tokens": n_prompt, "new_tokens": n_new, "dip_k": k, "hot_fraction": 0.2,
                     "model": "random-init Qwen3-1.7B shape, 28 layers, INT4 g128 linears, fp16 embed; LM head fp16 "
                              "(the reference's) or INT4 g128 (*_int4_head)",
                     "kv": "fp16, max_seq 2048"}
    return out


def decode_summary(dec: dict) -> dict:
    """Compact form of the decode record for the result line: tok/s per mode and the equality checks."""
    out = {m: v["decode_tok_s"] for m, v in dec.items() if isinstance(v, dict) and "decode_tok_s" in v}
    out.update({k: v for k, v in dec.items() if isinstance(v, bool)})
    return out


def entry(nbytes: int, us: float, **extra) -> dict:
    d = {"bytes": int(nbytes), "us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1),
         "frac_of_hbm": round(nbytes / (us * 1e-6) / HBM_PEAK, 4)}
    d.update(extra)
    return d


def bench_kernels(dev, gen):
    """Every hot-path kernel at its BASELINE shape (Qwen3-1.7B: H 2048, I 6144, 16/8 heads, hd 128),
    back-to-back launches replayed from a HIP graph over rotating copies of the large operands (>= 512 MB,
    past the 256 MB Infinity Cache). bytes = the algorithmic bytes each launch must move."""
    import torch

    from soinfer import _C, ops

    res = {}
    H, I, G = 2048, 6144, 2048 // GS
    row = H // 2
    f16, i32 = torch.float16, torch.int32

    # --- sparse down / indexed up / descriptors / fused GEMVs / device gather at k/I = 0.125 ... 0.5 ---
    n_cp = cold_copies(I * (row + 4 * G))
    Wt = [torch.randint(0, 256, (I, row), dtype=torch.uint8, device=dev, generator=gen) for _ in range(n_cp)]
    St = [(torch.rand(I, G, device=dev, generator=gen) * 0.01 + 1e-3) for _ in range(n_cp)]
    x = torch.randn(H, generator=gen, device=dev).half()
    gate = torch.randn(I, generator=gen, device=dev).half()
    for frac in (0.125, 0.25, 0.5):
        k = int(I * frac)
        idx = torch.sort(torch.randperm(I, device=dev, generator=gen)[:k]).values.to(i32)
        h = torch.randn(k, generator=gen, device=dev).half()
        y = torch.empty(H, dtype=f16, device=dev)
        ws = torch.zeros(max(1, _C.sparse_accumulate_workspace_bytes(H, k)), dtype=torch.uint8, device=dev)
        t = time_graph_per_launch(lambda W, S: _C.gemv_w4a16_indexed_accumulate_into(W, S, idx, h, y, H, GS, ws),
                                  list(zip(Wt, St)))
        res[f"sparse_down_k{k}"] = entry(k * (row + 4 * G + 2) + 2 * H, t["mean_us"],
                                         kernel="sparse_down (1 launch, last workgroup per slice sums)")
        u = torch.empty(k, dtype=f16, device=dev)
        t = time_graph_per_launch(lambda W, S: _C.gemv_w4a16_indexed_silu_into(W, S, idx, x, gate, u, H, GS),
                                  list(zip(Wt, St)))
        res[f"up_indexed_silu_k{k}"] = entry(k * (row + 4 * G + 4 + 2 + 2) + 2 * H, t["mean_us"],
                                             kernel="gemv_int4 IndexRows + SiLU epilogue")
        upv = torch.randn(I, generator=gen, device=dev).half()
        sel_i, sel_c = torch.empty(k, dtype=i32, device=dev), torch.empty(1, dtype=i32, device=dev)

        def two_launches(W, S):
            _C.topk_threshold_select_f16abs_into(gate, k, sel_i, sel_c)
            _C.gemv_w4a16_indexed_accumulate_gated_into(W, S, sel_i, gate, upv, y, H, GS, ws)

        t2 = time_graph_per_launch(two_launches, list(zip(Wt, St)))
        t = time_graph_per_launch(
            lambda W, S: _C.dip_select_gated_down_into(gate, upv, k, W, S, sel_i, sel_c, y, H, GS, ws),
            list(zip(Wt, St)))
        res[f"dip_select_gated_down_k{k}"] = entry(
            k * (row + 4 * G + 2 + 4) + 2 * I + 2 * H, t["mean_us"], two_launch_us=round(t2["mean_us"], 3),
            kernel="DIP selection over |gate| + gated sparse down (1 launch); two_launch_us: top-k, then gated down")
        dst = torch.empty(k, row, dtype=torch.uint8, device=dev)
        kcount = torch.full((1,), k, dtype=i32, device=dev)
        t = time_graph_per_launch(lambda W: _C.gather_rows_device_counted(W.data_ptr(), I, row, idx, kcount, dst),
                                  [(W,) for W in Wt])
        res[f"gather_rows_device_k{k}"] = entry(2 * k * row + 4 * k, t["mean_us"], kernel="gather_rows_device")
        if frac == 0.5:
            hot = torch.sort(torch.randperm(I, device=dev, generator=gen)[: int(0.2 * I)]).values
            slot_of = torch.full((I,), -1, dtype=i32, device=dev)
            slot_of[hot] = torch.arange(hot.numel(), dtype=i32, device=dev)
            desc, miss, mcount = torch.empty(k, dtype=i32, device=dev), torch.empty(k, dtype=i32, device=dev), \
                torch.empty(1, dtype=i32, device=dev)
            t = time_graph_per_launch(lambda: _C.build_dip_descriptors_into(idx, slot_of, desc, miss, mcount),
                                      [()] * 64)
            res[f"build_dip_descriptors_k{k}"] = entry(4 * k * 4 + 4, t["mean_us"], kernel="build_dip_descriptors")
            _C.build_dip_descriptors_into(idx, slot_of, desc, miss, mcount)
            mc = int(mcount.item())
            caches = [(W.index_select(0, hot).contiguous(), S.index_select(0, hot).contiguous()) for W, S in
                      zip(Wt, St)]
            stag = [(W.index_select(0, miss[:mc].long()).contiguous(), S.index_select(0, miss[:mc].long()).contiguous())
                    for W, S in zip(Wt, St)]
            args = [(c[0], c[1], st[0], st[1]) for c, st in zip(caches, stag)]
            t = time_graph_per_launch(lambda cW, cS, sW, sS: _C.gemv_dip_fused_up_into(cW, cS, sW, sS, desc, x, u, H,
                                                                                        GS), args)
            res[f"fused_up_k{k}"] = entry(k * (row + 4 * G + 4 + 2) + 2 * H, t["mean_us"], hot_fraction=0.2,
                                          kernel="gemv_int4 DescRows")
            t = time_graph_per_launch(lambda cW, cS, sW, sS: _C.gemv_dip_fused_down_into(cW, cS, sW, sS, desc, h, y,
                                                                                          H, GS, ws), args)
            res[f"fused_down_k{k}"] = entry(k * (row + 4 * G + 4 + 2) + 2 * H, t["mean_us"], hot_fraction=0.2,
                                            kernel="sparse_down DescRows (1 launch)")
            del caches, stag, args
    # the sparse down's fixed cost: k = 32 is one 32-row chunk per slice (8 workgroups, one arrival each), so the
    # time is the launch, one round trip of rows, the partial row, the arrival and the combine of a single row
    k = 32
    idx = torch.sort(torch.randperm(I, device=dev, generator=gen)[:k]).values.to(i32)
    h = torch.randn(k, generator=gen, device=dev).half()
    ws = torch.zeros(max(1, _C.sparse_accumulate_workspace_bytes(H, k)), dtype=torch.uint8, device=dev)
    t = time_graph_per_launch(lambda W, S: _C.gemv_w4a16_indexed_accumulate_into(W, S, idx, h, y, H, GS, ws),
                              list(zip(Wt, St)))
    res[f"sparse_down_k{k}"] = entry(k * (row + 4 * G + 2) + 2 * H, t["mean_us"],
                                     kernel="sparse_down (1 launch): the fixed cost of the arrival chain")
    # reads of pinned host rows through the device mapping (k = 3072 of the 6144 down^T rows, 6.3 MB arena):
    # whole 1 KB rows (the counted device gather) and the 128-byte row segments of the cached down with an empty
    # cache (every selected row a miss read in place)
    k = 3072
    idx = torch.sort(torch.randperm(I, device=dev, generator=gen)[:k]).values.to(i32)
    h = torch.randn(k, generator=gen, device=dev).half()
    host_W = Wt[0].cpu().pin_memory()
    addr = _C.host_device_pointer(host_W)
    kcount = torch.full((1,), k, dtype=i32, device=dev)
    dst = torch.empty(k, row, dtype=torch.uint8, device=dev)
    t = time_graph_per_launch(lambda: _C.gather_rows_device_counted(addr, I, row, idx, kcount, dst), [()] * 16)
    res[f"gather_rows_pinned_k{k}"] = {"bytes_over_pcie": k * row, "us": round(t["mean_us"], 3),
                                       "GBps": round(k * row / t["mean_us"] / 1e3, 2),
                                       "kernel": "gather_rows_device_counted from pinned host memory (1 KB rows)"}
    empty_W = torch.empty(0, row, dtype=torch.uint8, device=dev)
    empty_S = torch.empty(0, G, dtype=torch.float32, device=dev)
    slot_none = torch.full((I,), -1, dtype=i32, device=dev)
    ws = torch.zeros(max(1, _C.sparse_accumulate_workspace_bytes(H, k)), dtype=torch.uint8, device=dev)
    t = time_graph_per_launch(lambda: _C.gemv_dip_cached_down_into(empty_W, empty_S, host_W, St[0], slot_none, idx,
                                                                   h, y, H, GS, ws), [()] * 16)
    res[f"cached_down_all_miss_pinned_k{k}"] = {
        "bytes_over_pcie": k * row, "us": round(t["mean_us"], 3), "GBps": round(k * row / t["mean_us"] / 1e3, 2),
        "kernel": "sparse_down SlotRows, empty cache: every row read in place from pinned memory (128-byte "
                  "segments per workgroup)"}
    del host_W
    del Wt, St
    torch.cuda.empty_cache()

    # --- decode attention (host length and the engine's one-launch form) ---
    NQ, NKV, HD, S = 16, 8, 128, 2048
    n_cp = cold_copies(2 * NKV * S * HD * 2)
    KC = [torch.randn(NKV, S, HD, generator=gen, device=dev).half() for _ in range(n_cp)]
    VC = [torch.randn(NKV, S, HD, generator=gen, device=dev).half() for _ in range(n_cp)]
    q = torch.randn(NQ, HD, generator=gen, device=dev).half()
    qkv = torch.randn((NQ + 2 * NKV) * HD, generator=gen, device=dev).half()
    qn = torch.ones(HD, dtype=f16, device=dev)
    cos_t, sin_t = ops.rope_tables(HD, 1e6, S, dev)
    out = torch.empty(NQ, HD, dtype=f16, device=dev)
    ws_at = torch.zeros(_C.decode_attention_workspace_bytes(NQ, NKV, HD, S), dtype=torch.uint8, device=dev)
    ws_step = torch.zeros(_C.decode_attention_step_workspace_bytes(NQ, NKV, HD, S), dtype=torch.uint8, device=dev)
    WO = [torch.randint(0, 256, (2048, 1024), dtype=torch.uint8, device=dev, generator=gen) for _ in range(2)]
    SO = [torch.rand(2048, 16, device=dev, generator=gen) * 0.01 + 1e-3 for _ in range(2)]
    o_y = torch.empty(2048, dtype=f16, device=dev)
    for L in (192, 512, 2048):
        pos = torch.tensor([L - 1], dtype=i32, device=dev)
        nb = 4096 * L + 8192
        t = time_graph_per_launch(lambda kc, vc: _C.decode_attention_at(q, kc, vc, pos, out, ws_at),
                                  list(zip(KC, VC)))
        res[f"attention_L{L}"] = entry(nb, t["mean_us"], kernel="attn_kernel, device position (1 launch)")
        t = time_graph_per_launch(lambda kc, vc: _C.decode_attention_into(q, kc, vc, L, out, ws_at),
                                  list(zip(KC, VC)))
        res[f"attention_host_L{L}"] = entry(
            nb, t["mean_us"], kernel="attn_kernel, host length (the reference operator's form): a split context "
                                     "leaves its states to attn_combine_kernel (2 launches)")
        t = time_graph_per_launch(lambda kc, vc: _C.decode_attention_step(qkv, qn, qn, cos_t, sin_t, pos, kc, vc, out,
                                                                          1e-6, ws_step), list(zip(KC, VC)))
        res[f"attention_step_L{L}"] = entry(nb + 2 * (NQ + 2 * NKV) * HD, t["mean_us"],
                                            kernel="attn_kernel with q/k norm + RoPE + KV append (1 launch)")
        # the engine's pair: attention step, then the o projection (2048 x 2048 INT4) on its output; deferred:
        # the split states combined by the o projection while its weights load
        args = [(kc, vc, W, Sc) for (kc, vc), (W, Sc) in zip(zip(KC, VC), zip(WO * len(KC), SO * len(KC)))]
        t = time_graph_per_launch(lambda kc, vc, W, Sc: (
            _C.decode_attention_step(qkv, qn, qn, cos_t, sin_t, pos, kc, vc, out, 1e-6, ws_step),
            _C.gemv_w4a16_into(W, Sc, out.view(-1), o_y, NQ * HD, GS)), args)
        nbo = nb + 2 * (NQ + 2 * NKV) * HD + 2048 * 1024 + 2048 * 16 * 4 + 2 * 2048
        res[f"attention_step_o_L{L}"] = entry(nbo, t["mean_us"], kernel="attn_kernel step + o GEMV (2 launches)")
        t = time_graph_per_launch(lambda kc, vc, W, Sc: (
            _C.decode_attention_step_deferred(qkv, qn, qn, cos_t, sin_t, pos, kc, vc, out, 1e-6, ws_step),
            _C.gemv_w4a16_attn_combine_into(W, Sc, ws_step, out, pos, NKV, S, o_y, GS)), args)
        res[f"attention_step_deferred_o_L{L}"] = entry(
            nbo, t["mean_us"], kernel="attn_kernel step leaving split states + o GEMV combining them on load "
                                      "(2 launches)")
        t = time_graph_per_launch(lambda kc, vc: _C.decode_attention_step_deferred(qkv, qn, qn, cos_t, sin_t, pos, kc,
                                                                                   vc, out, 1e-6, ws_step),
                                  list(zip(KC, VC)))
        res[f"attention_step_deferred_L{L}"] = entry(
            nb + 2 * (NQ + 2 * NKV) * HD, t["mean_us"],
            kernel="attn_kernel step leaving a split context's states to the o projection (1 launch)")
    del KC, VC
    torch.cuda.empty_cache()

    # --- LM head (fp16 151936 x 2048) and argmax ---
    V = 151936
    n_cp = max(2, cold_copies(V * H * 2))
    LM = [torch.randn(V, H, generator=gen, device=dev).half() for _ in range(n_cp)]
    logits = torch.empty(V, dtype=f16, device=dev)
    t = time_graph_per_launch(lambda W: _C.gemv_f16_into(W, x, logits), [(W,) for W in LM])
    res["lm_head_fp16_gemv"] = entry(V * H * 2 + 2 * H + 2 * V, t["mean_us"], kernel="gemv_f16")
    del LM
    # the INT4 g128 head (config 5's "all weights INT4"): the same INT4 GEMV as every linear, 151936 rows
    n_cp = max(2, cold_copies(V * (row + 4 * G)))
    LQ = [(torch.randint(0, 256, (V, row), dtype=torch.uint8, device=dev, generator=gen),
           torch.rand(V, G, device=dev, generator=gen) * 0.01 + 1e-3) for _ in range(n_cp)]
    t = time_graph_per_launch(lambda W, S: _C.gemv_w4a16_into(W, S, x, logits, H, GS), LQ)
    res["lm_head_int4_gemv"] = entry(V * (row + 4 * G) + 2 * H + 2 * V, t["mean_us"], kernel="gemv_int4 (StoreY)")
    del LQ
    tok = torch.empty(1, dtype=i32, device=dev)
    aws = torch.empty(_C.argmax_workspace_bytes(V), dtype=torch.uint8, device=dev)
    t = time_graph_per_launch(lambda: _C.argmax_f16_into(logits, tok, None, None, aws), [()] * 64)
    res["argmax_vocab"] = entry(2 * V + 4, t["mean_us"], kernel="argmax partial + final (2 launches)")
    torch.cuda.empty_cache()

    # --- fused decode-step GEMVs (RMSNorm on load; SwiGLU epilogue) ---
    for name, N, swiglu in (("qkv_rmsnorm_4096x2048", 4096, False), ("gate_up_swiglu_12288x2048", 12288, True)):
        n_cp = cold_copies(N * (row + 4 * G))
        Ws = [torch.randint(0, 256, (N, row), dtype=torch.uint8, device=dev, generator=gen) for _ in range(n_cp)]
        Ss = [(torch.rand(N, G, device=dev, generator=gen) * 0.01 + 1e-3) for _ in range(n_cp)]
        d = torch.randn(H, generator=gen, device=dev).half()
        yy = torch.empty(N // 2 if swiglu else N, dtype=f16, device=dev)
        xo = torch.empty(H, dtype=f16, device=dev)
        nw = torch.ones(H, dtype=f16, device=dev)
        t = time_graph_per_launch(lambda W, S: _C.gemv_w4a16_rmsnorm_into(W, S, x, d, nw, 1e-6, xo, None, yy, H, GS,
                                                                          swiglu), list(zip(Ws, Ss)))
        res[name] = entry(N * (row + 4 * G) + 3 * 2 * H + 2 * yy.numel(), t["mean_us"],
                          kernel="gemv_int4_norm (residual add + RMSNorm on load" + (", SwiGLU epilogue)" if swiglu
                                                                                      else ")"))
        del Ws, Ss
        torch.cuda.empty_cache()

    # --- the resident DIP schedule's two MLP launches: gate|up GEMV with RMSNorm and SwiGLU that also stores the
    # gate of every channel; the rule-A selection + down as one dense GEMV over the transposed down_proj^T ---
    N = 2 * I
    n_cp = cold_copies(N * (row + 4 * G))
    Ws = [torch.randint(0, 256, (N, row), dtype=torch.uint8, device=dev, generator=gen) for _ in range(n_cp)]
    Ss = [(torch.rand(N, G, device=dev, generator=gen) * 0.01 + 1e-3) for _ in range(n_cp)]
    d = torch.randn(H, generator=gen, device=dev).half()
    nw = torch.ones(H, dtype=f16, device=dev)
    g_all, h_all = torch.empty(I, dtype=f16, device=dev), torch.empty(I, dtype=f16, device=dev)
    t = time_graph_per_launch(lambda W, S: _C.gemv_w4a16_rmsnorm_swiglu_gate_into(W, S, x, d, nw, 1e-6, None, g_all,
                                                                                  h_all, H, GS), list(zip(Ws, Ss)))
    res["gate_up_swiglu_gate_12288x2048"] = entry(N * (row + 4 * G) + 3 * 2 * H + 2 * 2 * I, t["mean_us"],
                                                  kernel="gemv_int4_norm (RMSNorm on load, SwiGLU epilogue storing "
                                                         "gate and h of every channel)")
    del Ws, Ss
    torch.cuda.empty_cache()
    n_cp = cold_copies(H * (I // 2 + 4 * I // GS))
    Wd = [torch.randint(0, 256, (H, I // 2), dtype=torch.uint8, device=dev, generator=gen) for _ in range(n_cp)]
    Sd = [(torch.rand(H // GS, I, device=dev, generator=gen) * 0.01 + 1e-3) for _ in range(n_cp)]
    g_all.copy_(torch.randn(I, generator=gen, device=dev).half())
    h_all.copy_(torch.randn(I, generator=gen, device=dev).half())
    yd = torch.empty(H, dtype=f16, device=dev)
    for k in (768, 3072):
        t = time_graph_per_launch(lambda W, S: _C.dip_select_dense_down_into(g_all, h_all, k, W, S, None, None, yd, GS),
                                  list(zip(Wd, Sd)))
        res[f"dip_dense_down_k{k}"] = entry(H * I // 2 + 4 * (H // GS) * I + 4 * I + 2 * H, t["mean_us"],
                                            kernel="dip_dense_down (rule-A selection in every workgroup + the down "
                                                   "as one GEMV over the transposed down_proj^T, 1 launch)")
        t = time_graph_per_launch(lambda W, S: _C.dip_select_down_ordered_into(g_all, h_all, k, W, S, None, None, yd,
                                                                                GS), list(zip(Wd, Sd)))
        res[f"dip_select_down_ordered_k{k}"] = entry(
            H * I // 2 + 4 * (H // GS) * I + 4 * I + 2 * H, t["mean_us"],
            kernel="dip_down_ordered (rule-A selection in every workgroup + the sparse down of the selected channels "
                   "in its own order, over the transposed down_proj^T, 1 launch)")
    del Wd, Sd
    torch.cuda.empty_cache()

    # --- host gathers from pinned memory (R8: the reference's staged vs per-row forms), wall clock incl. sync ---
    host = torch.randint(0, 256, (I, row), dtype=torch.uint8, generator=torch.Generator().manual_seed(5)).pin_memory()
    staging = torch.empty(I * row, dtype=torch.uint8).pin_memory()
    for k in (768, 3072):
        sel = torch.sort(torch.randperm(I, generator=torch.Generator().manual_seed(k))[:k]).values
        dst = torch.empty(k, row, dtype=torch.uint8, device=dev)
        for name, fn in (("staged", lambda: ops.gather_rows_staged(host, sel, staging, dst)),
                         ("naive", lambda: ops.gather_rows_naive(host, sel, dst))):
            fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(10):
                fn()
                torch.cuda.synchronize()
            us = (time.perf_counter() - t0) / 10 * 1e6
            res[f"gather_rows_{name}_k{k}"] = {"bytes": k * row, "us": round(us, 2),
                                               "GBps": round(k * row / us / 1e3, 2),
                                               "kernel": f"gather_rows_{name} (host pinned -> device, synchronized)"}
        assert torch.equal(dst.cpu(), host[sel]), "host gather bytes"
    del host, staging
    return res


def bench_grid_barrier(dev):
    """The cost of one grid-wide barrier among P co-resident workgroups (csrc/grid_sync.hip: O(P) arrival over
    8 per-XCD counters and a global one, one polling lane per workgroup, data exchanged device-coherent; and the
    same with an agent-scope release / acquire pair), against the boundary between two dependent launches of a
    captured graph, which is what a persistent decode launch would replace by such a barrier. Per barrier:
    (span of 201 rounds - span of 1 round) / 200, best of 5, from s_memrealtime stamps."""
    import torch

    from soinfer import _C

    out = {}
    maxp = _C.grid_barrier_max_workgroups()
    for fenced in (False, True):
        for P in (256, 1024):
            if P > maxp:
                continue
            ws = torch.zeros(_C.grid_barrier_bench_workspace_bytes(P), dtype=torch.uint8, device=dev)
            spans = {}
            for rounds in (1, 201):
                best = None
                for _ in range(5):
                    _C.grid_barrier_bench(fenced, P, rounds, ws)
                    torch.cuda.synchronize()
                    st = ws[4608:4608 + 16 * P].view(torch.int64).view(P, 2).cpu()
                    span = int((st[:, 1].max() - st[:, 0].min()).item()) * 10  # 100 MHz stamps -> ns
                    best = span if best is None else min(best, span)
                spans[rounds] = best
            err = ws[:4608].view(torch.int32)[1088:1090].tolist()
            assert err == [0, 0], f"grid barrier: timeout flag / mismatches {err}"
            out[f"{'fenced_' if fenced else ''}P{P}_us"] = round((spans[201] - spans[1]) / 200 / 1e3, 3)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    out["graph_launch_boundary_us"] = round(graph_time_us(lambda: [_C.advance_position(pos, 1) for _ in range(100)])
                                            / 100, 3)
    out["note"] = ("P workgroups of 256 threads; per barrier = (201 rounds - 1 round) / 200. A persistent decode launch "
                   "would replace each graph launch boundary by one such barrier (plus the device-coherent reload of "
                   "the exchanged vector), so it cannot beat the launch chain")
    return out


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def _time_passes(fn, warmup: int = 20, iters: int = 100):
    """median and p90 (seconds) of `iters` timed calls of fn after `warmup` untimed ones (bench/harness.py:36-74
    of the reference: >= 20 warmup, >= 100 iterations)."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], ts[min(len(ts) - 1, int(0.9 * len(ts)))]


def cpu_baseline(layer0):
    """The reference's CPU GEMV path (formats.dequantize, then fp32 torch.mv, rounded to fp16:
    tests/test_m4_kernels.py:157-165, restated in oracle/cpu_path.py) over layer 0's seven GEMVs, one pass = all
    seven, timed with 20 warmup and 100 timed passes (median and p90) on the host cores this job may use (at most
    16, the box's CPU share for one GPU) and on one thread; beside it the matmul alone on pre-dequantized fp32
    weights, and the C oracle's binary64 GEMV (the tests' checker) for reference. layer0: (q int8 [N, K],
    scale fp32 [N, K/gs], Wq packed, x fp16 [K], K) per GEMV."""
    import torch

    from oracle import cpu_path
    from oracle import oracle as O

    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cores = max(1, min(16, avail))
    qs = [(torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(x), K) for q, s, _, x, K in layer0]
    pass_bytes = sum(int4_bytes(q.shape[0], K) for q, _, _, K in qs)
    pre = [cpu_path.dequantize_group(q, s, K, GS) for q, s, _, K in qs]

    def dequant_mv():
        for q, s, x, K in qs:
            cpu_path.gemv_dequant_mv(q, s, x, K, GS)

    def mv_only():
        for W, (_, _, x, _) in zip(pre, qs):
            cpu_path.gemv_mv_predequantized(W, x)

    # the other hot-path operators' CPU oracles of the reference's tests (oracle/cpu_path.py) at the BASELINE
    # shapes: top-k over |gate| I = 6144, k = 3072; gather of 3072 1 KB rows; sparse down over 3072 selected rows
    # of down^T (pre-dequantized, and with the dequantize of the selected rows); attention at L = 192 and 2048
    gen = torch.Generator().manual_seed(11)
    I, H, kk = 6144, 2048, 3072
    abs_g = torch.randn(I, generator=gen).half().float().abs()
    rows = torch.randint(0, 256, (I, H // 2), dtype=torch.uint8, generator=gen)
    sel = torch.sort(torch.randperm(I, generator=gen)[:kk]).values
    q_d = torch.randint(-7, 8, (kk, H), dtype=torch.int8, generator=gen)
    s_d = torch.rand(kk, H // GS, generator=gen) * 0.01
    h_sel = torch.randn(kk, generator=gen).half()
    Wd_sel = cpu_path.dequantize_group(q_d, s_d, H, GS)
    qa = torch.randn(16, 128, generator=gen).half()
    kc, vc = torch.randn(8, 2048, 128, generator=gen).half(), torch.randn(8, 2048, 128, generator=gen).half()
    others = (("topk_I6144_k3072", lambda: cpu_path.topk_indices(abs_g, kk)),
              ("gather_rows_k3072", lambda: cpu_path.gather_rows(rows, sel)),
              ("sparse_down_k3072_predequantized", lambda: cpu_path.sparse_accumulate_ref(h_sel, Wd_sel)),
              ("sparse_down_k3072_with_dequantize",
               lambda: cpu_path.sparse_accumulate_ref(h_sel, cpu_path.dequantize_group(q_d, s_d, H, GS))),
              ("attention_L192", lambda: cpu_path.decode_attention_ref(qa, kc, vc, 192)),
              ("attention_L2048", lambda: cpu_path.decode_attention_ref(qa, kc, vc, 2048)))

    saved = torch.get_num_threads()
    figures, other_figures = {}, {}
    try:
        for threads in (cores, 1):
            torch.set_num_threads(threads)
            for name, fn in (("dequant_mv", dequant_mv), ("mv_predequantized", mv_only)):
                med, p90 = _time_passes(fn)
                figures[f"{name}_{threads}t"] = {"median_ms": round(med * 1e3, 3), "p90_ms": round(p90 * 1e3, 3),
                                                 "GBps": round(pass_bytes / med / 1e9, 4)}
            for name, fn in others:
                med, p90 = _time_passes(fn)
                other_figures[f"{name}_{threads}t"] = {"median_us": round(med * 1e6, 1), "p90_us": round(p90 * 1e6, 1)}
    finally:
        torch.set_num_threads(saved)

    # the binary64 scalar C checker, a bounded sample
    t0, reps = time.perf_counter(), 0
    while time.perf_counter() - t0 < 2.0:
        for q, s, Wq, x, K in layer0:
            O.gemv_w4_f64(Wq, s, x, K, GS, threads=cores)
        reps += 1
    checker = round(reps * pass_bytes / (time.perf_counter() - t0) / 1e9, 4)
    main_fig = figures[f"dequant_mv_{cores}t"]
    short = (f"reference CPU GEMV path (formats.dequantize + fp32 torch.mv, tests/test_m4_kernels.py:157-165; "
             f"oracle/cpu_path.py) over layer 0's 7 INT4 g128 GEMVs, {pass_bytes} B per pass, median of 100 passes "
             f"at {cores} threads; {_cpu_model()}")
    return {"value": main_fig["GBps"], "short_sample": short, "unit": "GB/s", "cores": cores, "kind": "port",
            "median_ms_per_pass": main_fig["median_ms"], "p90_ms_per_pass": main_fig["p90_ms"],
            "single_thread_value": figures["dequant_mv_1t"]["GBps"], "figures": figures,
            "c_oracle_binary64_GBps": checker, "other_operators": other_figures,
            "sample": f"the reference's CPU GEMV path (formats.dequantize of the int8 codes and fp32 scales, then "
                      f"fp32 torch.mv, fp16 out; tests/test_m4_kernels.py:157-165, restated in oracle/cpu_path.py) "
                      f"over layer 0's 7 INT4 g128 GEMVs ({pass_bytes} algorithmic bytes per pass), 20 warmup + 100 "
                      f"timed passes, median, torch.set_num_threads({cores}); GB/s = algorithmic INT4 bytes / "
                      f"time, as the GPU figure. Also: 1 thread, the matmul alone on pre-dequantized fp32, and "
                      f"the C oracle's binary64 GEMV (the tests' checker, not the baseline). other_operators: the "
                      f"reference tests' CPU oracles of the other path operators (torch.topk, index_select, "
                      f"h @ W_dequant, decode_attention_ref; oracle/cpu_path.py) at the BASELINE shapes, 20 warmup + "
                      f"100 timed calls, median and p90 in us. Host: {_cpu_model()}, "
                      f"{avail} cores available to the job"}


def run_traffic_set(dev, gen):
    """Launches for the HBM counter passes (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, one run each): the
    calibration copy (copy_reference: 11 copies of 512 MiB), then 6 launches each, on separate operand copies
    and each followed by a synchronize, of sparse_down_kernel, dip_select_down_kernel and dip_dense_down_kernel
    (index list not written) at k = 3072 and of attn_kernel at L = 192 and L = 2048 (host-length form, one
    workgroup per query head: grids of 16 and 16 x 16 workgroups, the latter followed by attn_combine_kernel over
    the split states). Prints the algorithmic bytes each launch moves."""
    import torch

    from soinfer import _C

    copy_reference()
    H, I, G = 2048, 6144, 2048 // GS
    row = H // 2
    f16, i32 = torch.float16, torch.int32
    n = 6
    Wt = [torch.randint(0, 256, (I, row), dtype=torch.uint8, device=dev, generator=gen) for _ in range(n)]
    St = [(torch.rand(I, G, device=dev, generator=gen) * 0.01 + 1e-3) for _ in range(n)]
    k = 3072
    idx = torch.sort(torch.randperm(I, device=dev, generator=gen)[:k]).values.to(i32)
    h = torch.randn(k, generator=gen, device=dev).half()
    y = torch.empty(H, dtype=f16, device=dev)
    ws = torch.zeros(_C.sparse_accumulate_workspace_bytes(H, k), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    for W, S in zip(Wt, St):
        _C.gemv_w4a16_indexed_accumulate_into(W, S, idx, h, y, H, GS, ws)
        torch.cuda.synchronize()
    gate = torch.randn(I, generator=gen, device=dev).half()
    up = torch.randn(I, generator=gen, device=dev).half()
    sel_i, sel_c = torch.empty(k, dtype=i32, device=dev), torch.empty(1, dtype=i32, device=dev)
    for W, S in zip(Wt, St):
        _C.dip_select_gated_down_into(gate, up, k, W, S, sel_i, sel_c, y, H, GS, ws)
        torch.cuda.synchronize()
    del Wt, St
    # dip_dense_down_kernel: the transposed copy of the whole down^T ([H, I/2] nibbles, [G, I] scales)
    Wd = [torch.randint(0, 256, (H, I // 2), dtype=torch.uint8, device=dev, generator=gen) for _ in range(n)]
    Sd = [(torch.rand(G, I, device=dev, generator=gen) * 0.01 + 1e-3) for _ in range(n)]
    hd = torch.randn(I, generator=gen, device=dev).half()
    torch.cuda.synchronize()
    for W, S in zip(Wd, Sd):
        _C.dip_select_dense_down_into(gate, hd, k, W, S, None, None, y, GS)
        torch.cuda.synchronize()
    del Wd, Sd
    NQ, NKV, HD, Smax = 16, 8, 128, 2048
    q = torch.randn(NQ, HD, generator=gen, device=dev).half()
    for L in (192, 2048):
        for _ in range(n):
            kc = torch.randn(NKV, Smax, HD, generator=gen, device=dev).half()
            vc = torch.randn(NKV, Smax, HD, generator=gen, device=dev).half()
            torch.cuda.synchronize()
            _C.decode_attention(q, kc, vc, L)
            torch.cuda.synchronize()
    print(json.dumps({"traffic_set": {
        "sparse_down_kernel_k3072": {"read": k * (row + 4 * G + 2 + 4), "write": 2 * H},
        "dip_select_down_kernel_k3072": {"read": k * (row + 4 * G + 2) + 2 * I, "write": 2 * H + 4 * k + 4},
        "dip_dense_down_kernel_k3072": {"read": H * I // 2 + 4 * G * I + 2 * I + 2 * I, "write": 2 * H},
        "attn_kernel_L192": {"read": 4096 * 192 + 2 * NQ * HD, "write": 2 * NQ * HD},
        "attn_kernel_L2048": {"read": 4096 * 2048 + 2 * NQ * HD, "write": 2 * NQ * HD}}}))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ramp-ms", type=float, default=250.0,
                    help="untimed streaming of the weight set before the warmup steps (ms of wall time)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the decode-chain, per-shape and top-k tables")
    ap.add_argument("--no-decode", action="store_true", help="skip the DIP MLP and decode tok/s sections")
    ap.add_argument("--detail-json", default=None, help="also write the result and the detail record to this file")
    ap.add_argument("--traffic-set", action="store_true",
                    help="only the launches of the HBM counter passes (calibration copy, sparse down, fused "
                         "selection + down, dense down, attention at L = 192 and 2048), then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU (the hot path is single-GPU; --gpus {args.gpus} is not "
              "supported). Run with --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from __graft_entry__ import ensure_built

    ensure_built()
    import soinfer.ops as ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    if args.traffic_set:
        run_traffic_set(dev, gen)
        return 0

    # ---- the 28-layer weight set, resident in HBM ----
    layers = []
    step_bytes = 0
    for layer in range(LAYERS):
        mats = {}
        for name, N, K in LAYER_SHAPES:
            Wq, s = make_int4(N, K, gen, dev)
            x = torch.randn(K, generator=gen, device=dev).half()
            mats[name] = (Wq, s, x, N, K)
            step_bytes += int4_bytes(N, K)
        layers.append(mats)
    torch.cuda.synchronize()
    log(f"weight set ready: {LAYERS} layers, {step_bytes} bytes per step")

    # One step = every GEMV of the weight set, all 196 in ONE grouped launch
    # (4 shape classes; the long-row down class is laid out first).
    order = [(l, n) for l in range(LAYERS) for n, _, _ in LAYER_SHAPES]
    group = ops.GemvGroup([(layers[l][n][0], layers[l][n][1], layers[l][n][2], layers[l][n][4]) for l, n in order], GS)

    def step():
        group.run()

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    # the same number of steps before the ramp (detail record only: the cold-start rate)
    ev_c0, ev_c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev_c0.record()
    for _ in range(args.steps):
        step()
    ev_c1.record()
    ev_c1.synchronize()
    cold_us = ev_c0.elapsed_time(ev_c1) * 1e3 / args.steps
    # load ramp: the first launches after set-up run slower than the loaded steady state (the same 50 steps after
    # 5 / 50 / 200 / 1000 warmup steps: 130.9 / 129.0 / 119.0 / 116.8 us per launch, one box), so the weight set
    # is streamed for --ramp-ms of wall time (untimed) before the W warmup steps
    ramp_steps = 0
    t_ramp = time.perf_counter()
    while (time.perf_counter() - t_ramp) * 1e3 < args.ramp_ms:
        for _ in range(16):
            step()
        torch.cuda.synchronize()
        ramp_steps += 16
    log(f"{args.steps} steps before the ramp: {cold_us:.3f} us per launch (events); load ramp: {ramp_steps} untimed "
        f"steps in {(time.perf_counter() - t_ramp) * 1e3:.0f} ms")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # the timed region: wall clock between two device synchronisations, and two HIP events on the launching
    # (current) stream around the same launches, so the dominant kernel's average duration comes from the
    # very launches ms_per_step times (one launch per step)
    ev_a, ev_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev_a.record()
    for _ in range(args.steps):
        step()
    ev_b.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    dom_us = ev_a.elapsed_time(ev_b) * 1e3 / args.steps
    log(f"{args.steps} timed steps: {elapsed / args.steps * 1e3:.4f} ms/step, {dom_us:.3f} us per launch (events)")
    ms_per_step = elapsed / args.steps * 1e3
    value = step_bytes / (elapsed / args.steps) / 1e9  # GB/s

    # per-step spread, measured after the timed region (HIP events around each of 100 steps)
    per_step = []
    for _ in range(100):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        step()
        b.record()
        b.synchronize()
        per_step.append(a.elapsed_time(b) * 1e3)
    per_step.sort()
    step_stats = {"median_us": round(per_step[50], 2), "p90_us": round(per_step[90], 2),
                  "min_us": round(per_step[0], 2), "note": "100 steps, each timed alone (idle gap between steps)"}

    # the grouped outputs equal single launches (spot checks, bit-exact)
    for i in (0, 4, 6, len(order) - 1):
        l, n = order[i]
        m = layers[l][n]
        assert torch.equal(group.ys[i], ops.gemv_w4a16_group_lop3(m[0], m[1], m[2], m[4], GS)), f"grouped {l}.{n}"

    # ---- dominant kernel: the grouped launch (the whole step), from the events around the timed steps ----
    achieved = step_bytes / (dom_us * 1e-6) / 1e9
    n_wg = sum(c * (nn // 8) for c, nn in zip(group.class_count, group.class_N))
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(achieved * 1e9 / HBM_PEAK, 4), "traffic": read_traffic(),
                "kernel": f"soi::gemv_int4_grouped_occ_kernel<8,true,true,true> (196 GEMVs in 4 shape classes, "
                          f"{n_wg} workgroups of 64)",
                "bytes_per_launch": step_bytes, "avg_launch_us": round(dom_us, 3),
                "timing": f"HIP events on the launching stream around the {args.steps} timed steps (one launch "
                          f"each)"}
    # after the timed region: 30 more back-to-back launches, for the detail record only
    dom_b2b_us = time_back_to_back(group.run, launches=30)
    log(f"dominant launch after the timed region: {dom_b2b_us:.3f} us")

    # ---- the same work as one batched launch per shape class (4 launches), per class ----
    per_class = {}
    for names in (("down",), ("gate", "up"), ("q", "o"), ("k", "v")):
        mats = [layers[l][n] for l in range(LAYERS) for n in names]
        N, K = mats[0][3], mats[0][4]
        bt = ops.GemvBatch([m[0] for m in mats], [m[1] for m in mats], [m[2] for m in mats], K, GS)
        us = time_back_to_back(bt.run, launches=20)
        nbytes = len(mats) * int4_bytes(N, K)
        per_class["/".join(names)] = {"problems": len(mats), "N": N, "K": K, "bytes": nbytes, "us": round(us, 3),
                                      "GBps": round(nbytes / us / 1e3, 1),
                                      "frac_of_hbm": round(nbytes / (us * 1e-6) / HBM_PEAK, 4)}
        del bt
    log("per-class batched launches done")
    # the INT8 g128 half of config 2 at the same scale: one batched launch per shape over 28 (down) or 56 distinct
    # weight copies (the quantized values of one matrix per shape, copied: the bytes, not the values, matter here)
    int8_per_class = {}
    for names, N, K in ((("down",), H, I), (("gate", "up"), I, H), (("q", "o"), NQ * HD, H), (("k", "v"), NKV * HD, H)):
        P = LAYERS * len(names)
        q8, s8 = make_int8(N, K, gen, dev)
        Q8 = [q8.clone() for _ in range(P)]
        S8 = [s8.clone() for _ in range(P)]
        X8 = [torch.randn(K, generator=gen, device=dev).half() for _ in range(P)]
        b8 = ops.Int8Batch(Q8, S8, X8, GS)
        us = time_back_to_back(b8.run, launches=20)
        nbytes = P * int8_bytes(N, K)
        int8_per_class["/".join(names)] = {"problems": P, "N": N, "K": K, "bytes": nbytes, "us": round(us, 3),
                                           "GBps": round(nbytes / us / 1e3, 1),
                                           "frac_of_hbm": round(nbytes / (us * 1e-6) / HBM_PEAK, 4)}
        del Q8, S8, X8, b8
    torch.cuda.empty_cache()
    log("INT8 per-class batched launches done")
    copy_ref = copy_reference()
    # the same copy at the sizes the kernels here move: one gate/up GEMV's bytes, 64 MB, and a whole step
    copy_ref["by_size"] = {str(nb): copy_reference(nb, reps=30 if nb < (256 << 20) else 10)
                           for nb in (int4_bytes(6144, 2048), 64 << 20, step_bytes)}
    log(f"copy reference: {copy_ref['us']} us")


    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic: W ~ N(0,0.02) quantized INT4 g128 (fp32 scales), x ~ N(0,1) fp16, seeded",
        "config": {"workload": "INT4 g128 GEMV sweep at batch 1 over all 196 linear weights of a 28-layer "
                               "Qwen3-1.7B-shaped decoder (q,k,v,o,gate,up,down; each GEMV its own x), HBM-resident; "
                               "all 196 GEMVs in one grouped launch per step",
                   "bytes_per_step": step_bytes, "layers": LAYERS, "hidden": H, "intermediate": I,
                   "group_size": GS, "ramp": f"{ramp_steps} untimed steps ({args.ramp_ms:g} ms) before the warmup"},
        "frac_of_hbm_peak": round(value * 1e9 / HBM_PEAK, 4),
        "roofline": roofline,
    }
    # everything else goes to the detail record (stderr, and --detail-json): the result line stays compact
    detail = {"dominant_launch_back_to_back_after_timed_us": round(dom_b2b_us, 3),
              "dominant_launch_before_ramp_us": round(cold_us, 3), "copy_reference": copy_ref,
              "batched_per_class": per_class, "int8_batched_per_class": int8_per_class, "step_spread": step_stats}
    if not args.no_extras:
        detail["decode_chain"] = bench_decode_chain(ops, layers, step_bytes)
        log("decode chain done")
        del layers, group
        torch.cuda.empty_cache()
        detail["per_shape_cold"] = bench_shapes(ops, dev, gen)
        log("per-shape table done")
        detail["topk_us_I6144"] = bench_topk(ops, dev, gen)
        log("top-k done")
        detail["kernels"] = bench_kernels(dev, gen)
        log("kernel table done")
        detail["grid_barrier"] = bench_grid_barrier(dev)
        log(f"grid barrier: {detail['grid_barrier']}")
    if not args.no_decode:
        from soinfer.runtime import decoder as D

        try:
            del layers, group
        except NameError:
            pass
        torch.cuda.empty_cache()
        w = D.random_decoder(D.QWEN3_1P7B, seed=0)
        calib = torch.randint(0, D.QWEN3_1P7B.vocab, (64,), generator=torch.Generator().manual_seed(1000)).tolist()
        from soinfer.offload.hot_cache import StaticFrequencyPolicy

        counts = D.calibrate_channel_counts(w, D.QWEN3_1P7B.intermediate // 2, calib)
        # hot sets as calibrate_hot_channels builds them (the most frequently selected channels), at the
        # config's 20% and, for the hot-fraction sweep, 50% and 100% of I
        hot_sets = {f: [StaticFrequencyPolicy(cnt.cpu(), int(round(f * D.QWEN3_1P7B.intermediate))).hot_indices
                        .tolist() for cnt in counts] for f in (0.2, 0.5, 1.0)}
        hot = hot_sets[0.2]
        del counts
        log("decoder weights and hot sets ready")
        detail["dip_mlp_layer"] = bench_dip_mlp(D, w, hot, dev)
        log("DIP MLP done")
        detail["decode"] = bench_decode(D, w, hot, dev, hot_sweep={"cached_dip_hot50": hot_sets[0.5],
                                                                    "cached_dip_hot100": hot_sets[1.0]})
        del w
        torch.cuda.empty_cache()
        result["decode_tok_s"] = decode_summary(detail["decode"])
    if not args.no_cpu_baseline:
        g = torch.Generator().manual_seed(1)
        layer0 = []
        from oracle import oracle as O

        for _, N, K in LAYER_SHAPES:
            q, s = O.quantize_group((torch.randn(N, K, generator=g) * 0.02).numpy(), GS)
            layer0.append((q, s, O.pack_int4(q), torch.randn(K, generator=g).half().numpy(), K))
        cpu = cpu_baseline(layer0)
        log("cpu baseline done")
        detail["cpu_baseline"] = cpu
        result["cpu_baseline"] = {k: cpu[k] for k in ("value", "unit", "cores", "kind", "single_thread_value",
                                                     "median_ms_per_pass")}
        result["cpu_baseline"]["sample"] = cpu["short_sample"]
    result["detail"] = "stderr line 'bench-detail: {...}' (and --detail-json)"
    dj = json.dumps(detail)
    print(f"bench-detail: {dj}", file=sys.stderr, flush=True)
    if args.detail_json:
        Path(args.detail_json).parent.mkdir(parents=True, exist_ok=True)
        Path(args.detail_json).write_text(json.dumps({"result": result, "detail": detail}, indent=1))
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
