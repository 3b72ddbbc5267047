"""Benchmark of the sparse-FFN decode hot path on one MI355X.

Default workload (one step = one decode token through one layer):
  Falcon-7B-shaped ReLU FFN layer, d_model=4544, d_ff=18176, Q4_0 weights in
  the bundled layout, rank-128 fp32 predictor, threshold giving ~5% (909)
  active neurons; each step runs predictor -> selection -> gathered up/down
  FFN on the device (llg_hipd_ffn_predict_sparse), with a fresh x per token.
  Steps rotate over LAYERS distinct HBM copies of the layer so that the
  gathered rows are not served from the 256 MB MALL.

Output: one JSON line (see the contract in the repository's docs), with a
`roofline` object for the sparse FFN kernels (algorithmic gathered bytes /
their average event-timed duration on the library's stream) and a
`cpu_baseline` object (the oracle's restatement of the reference CPU path,
timed on a bounded sample on this host).

The default run (--workload all) prints that line with every other workload
measured in the same process under its `workloads` key, each with its own
metric, roofline and, for the window and the full model, CPU baseline.  One
workload alone: --workload sparse | dense-q4_0 | dense-q8_0 | dense-f16 |
window | moe-decode | moe-prefill | falcon-decode | swiglu-q4_0 | swiglu-q8_0 |
swiglu-f16.  falcon-decode is the full 32-layer model around the sparse FFN
(--steps = generated tokens after the 512-token prompt); swiglu-* is the SiLU
architecture's dense FFN (ffnSwiGLU) at a LLaMA-7B layer's shape.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "llama.go_amd"))

HBM_PEAK_GBS = 8000.0
H, FF, RANK, N_ACTIVE = 4544, 18176, 128, 909
Q4_ROW = H // 32 * 18                # 2556 B per GGUF Q4_0 row
BUNDLE_ALG = 2 * Q4_ROW              # 5112 B per neuron (unpadded)
PRED_BYTES = (RANK * H + FF * RANK) * 4
# HBM bytes per sparse step from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE over
# k_tile_ffn (its predictor workgroups and tiles) + k_tile_reduce, each counter
# scaled by its reading for a 1 GiB streaming copy (FETCH x2.0, WRITE x1.0),
# measured on this bench
# line (exactly 909 active neurons per step): the weights once plus the
# workgroups' partial outputs written and read back; the summary with the
# commands is profiles/sparse_step_falcon7b_q4_0_hbm_traffic.md.
SPARSE_STEP_TRAFFIC = 22.28e6
SPARSE_STEP_TRAFFIC_ACTIVE = 909


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def vp(t) -> C.c_void_p:
    return C.c_void_p(t.data_ptr())


class Timer:
    """HIP events recorded on the library's own stream."""

    def __init__(self, torch, stream_ptr: int):
        self.torch = torch
        self.stream = torch.cuda.ExternalStream(stream_ptr)

    def event(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.stream)
        return e


def bench_sparse(args, torch, llg, dev):
    gg = llg.gguf
    L = args.layers
    log(f"sparse: generating layer on GPU (d={H}, ff={FF}, Q4_0), {L} HBM copies")
    g = torch.Generator(device="cuda")
    g.manual_seed(0x11A3A000)
    up = gg.quantize(torch.randn((FF, H), generator=g, device="cuda") * 0.02, gg.Q4_0)
    dn = gg.quantize(torch.randn((FF, H), generator=g, device="cuda") * 0.02, gg.Q4_0)
    wup = (torch.randn((RANK, H), generator=g, device="cuda") * 0.05).contiguous()
    wout = (torch.randn((FF, RANK), generator=g, device="cuda") * 0.05).contiguous()
    n_x = 64
    X, thrs = exact_active_inputs(torch, g, wup, wout, n_x)
    torch.cuda.synchronize()  # the library's stream does not wait on torch's
    bundles, wups, wouts = [], [], []
    for _ in range(L):
        bundles.append(dev.upload_bundle(up, dn, gg.Q4_0, H, FF))
        wups.append(dev.upload_matrix(wup, gg.F32, RANK, H))
        wouts.append(dev.upload_matrix(wout, gg.F32, FF, RANK))
    out = torch.empty((n_x, H), device="cuda")
    act = torch.empty((L, FF), dtype=torch.int32, device="cuda")
    nact = torch.zeros((L, 1), dtype=torch.int32, device="cuda")
    nstep = torch.zeros((max(args.steps, args.warmup) + 1, 1), dtype=torch.int32, device="cuda")
    lib = dev.lib

    def step(i):
        """ffnFlash path 2: predictor -> selection -> gathered FFN, 2 launches."""
        l = i % L
        x = X[i % n_x]
        rc = lib.llg_hipd_ffn_predict_sparse(dev.h, wups[l].id, wouts[l].id, 0, bundles[l].id,
                                             vp(x), vp(x), float(thrs[i % n_x]), gg.ACT_RELU,
                                             vp(out[i % n_x]), None, vp(nstep[i]))
        if rc:
            dev.check(rc, "ffn_predict_sparse")

    def ffn_only(i):
        """ffnSparseLoad over an explicit active list (k_list_up + k_sparse_down)."""
        l = i % L
        rc = lib.llg_hipd_ffn_sparse(dev.h, bundles[l].id, vp(X[l % n_x]), vp(act[l]),
                                     vp(nact[l]), gg.ACT_RELU, vp(out[i % n_x]))
        if rc:
            dev.check(rc, "ffn_sparse")

    def pred_only(i):
        """Predictor.Predict with the ascending active list (3 launches)."""
        l = i % L
        rc = lib.llg_hipd_predict(dev.h, wups[l].id, wouts[l].id, 0, vp(X[l % n_x]),
                                  float(thrs[l % n_x]), vp(act[l]), vp(nact[l]), None)
        if rc:
            dev.check(rc, "predict")

    tm = Timer(torch, dev.stream)
    for l in range(L):  # active lists for the list-path timing
        pred_only(l)
    for i in range(args.warmup):
        step(i)
    dev.sync()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    e0 = tm.event()
    for i in range(args.steps):
        step(i)
    e1 = tm.event()
    dev.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    mean_active = float(nstep[: args.steps].float().mean().item())

    def time_region(fn, n):
        a = tm.event()
        for i in range(n):
            fn(i)
        b = tm.event()
        dev.sync()
        return a.elapsed_time(b) / n

    ffn_ms = time_region(ffn_only, args.steps)
    pred_ms = time_region(pred_only, args.steps)
    list_active = float(nact.float().mean().item())
    for h_ in bundles + wups + wouts:
        h_.release()

    step_alg = PRED_BYTES + mean_active * BUNDLE_ALG
    step_gbs = step_alg / (ms_step * 1e-3) / 1e9
    ffn_alg = list_active * BUNDLE_ALG
    res = {
        "metric": "sparse-FFN decode tokens/s on 1 MI355X + achieved HBM GB/s vs 8 TB/s peak",
        "value": 1000.0 / ms_step,
        "unit": "tokens/s",
        "ms_per_step": ms_step,
        "dtype": "f32",
        "config": {"workload": "falcon7b-ffn-layer-q4_0-5pct-sparse-decode", "d_model": H,
                   "d_ff": FF, "predictor_rank": RANK, "weights": "Q4_0 bundled",
                   "target_active": N_ACTIVE, "mean_active": mean_active,
                   "threshold": "per token: fp32 midpoint of its 909th and 910th largest "
                                "predictor logit", "batch": 1,
                   "layer_copies_rotated": L, "step": "predict+select+gathered up/down FFN"},
        "roofline": {"bound": "hbm",
                     "kernel": "k_tile_ffn (predictor workgroups + tiles) + k_tile_reduce "
                               "(one decode step)",
                     "achieved": step_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": step_gbs / HBM_PEAK_GBS, "traffic": SPARSE_STEP_TRAFFIC,
                     "traffic_active_neurons": SPARSE_STEP_TRAFFIC_ACTIVE,
                     "alg_bytes_per_launch": step_alg, "avg_launch_us": ms_step * 1e3},
        "breakdown": {
            "ffn_list_path_us": ffn_ms * 1e3,
            "ffn_list_path_gbs": ffn_alg / (ffn_ms * 1e-3) / 1e9,
            "ffn_list_path_frac": ffn_alg / (ffn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "ffn_alg_bytes": ffn_alg, "list_mean_active": list_active,
            "predict_us": pred_ms * 1e3,
            "predict_gbs": PRED_BYTES / (pred_ms * 1e-3) / 1e9,
            "wall_s": wall},
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline_sparse(args, up.cpu().numpy(), dn.cpu().numpy(),
                                                  wup.cpu().numpy(), wout.cpu().numpy(),
                                                  X.cpu().numpy(), thrs)
    return res


def exact_active_inputs(torch, g, wup, wout, n_x):
    """n_x inputs x ~ N(0, 1) and, per input, the threshold that activates
    exactly N_ACTIVE neurons: the fp32 midpoint of its N_ACTIVE-th and
    (N_ACTIVE+1)-th largest predictor logit (float64 on the device).  Inputs
    whose two logits lie closer than 1e-4 of the logits' standard deviation
    are skipped, so that fp32 reordering in the kernels cannot move a neuron
    across the threshold."""
    cand = torch.randn((2 * n_x, H), generator=g, device="cuda")
    hid = torch.relu(wup.double() @ cand.double().T)        # [rank, 2 n_x]
    lg = wout.double() @ hid                                 # [FF, 2 n_x]
    top = torch.topk(lg, N_ACTIVE + 1, dim=0).values
    a, b = top[N_ACTIVE - 1], top[N_ACTIVE]
    keep = torch.nonzero((a - b) > 1e-4 * lg.std(dim=0)).flatten()[:n_x]
    if keep.numel() < n_x:
        raise RuntimeError("too few inputs with a clear 909/910 logit gap")
    thrs = ((a + b) / 2)[keep].float().cpu().numpy()
    return cand[keep].contiguous(), thrs


def usable_cpus() -> int:
    """The host CPUs this process may run on (its affinity mask)."""
    return len(os.sched_getaffinity(0))


def host_cpu() -> dict:
    """The host's CPU model, its logical CPUs and those this process may use."""
    model = "unknown"
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "usable_cpus": usable_cpus(), "cpu_model": model}


def layer_file(up, dn, t):
    """Write ffn_up and the transposed ffn_down (GGUF dims [h, F], one row per
    neuron) to a GGUF file in the temp directory and read it once, so that it
    sits in the page cache as the reference's weights do after the first
    token.  Returns (path, up offset, down offset)."""
    import tempfile

    from llg import gguf_file as GF

    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    GF.write_gguf(path, [("general.architecture", GF.T_STRING, "falcon")],
                  [("blk.0.ffn_up.weight", [H, FF], t, up),
                   ("blk.0.ffn_down_t.weight", [H, FF], t, dn)])
    with open(path, "rb") as f:
        while f.read(1 << 24):
            pass
    gf = GF.open_gguf(path)
    return (path, gf.by_name["blk.0.ffn_up.weight"].offset,
            gf.by_name["blk.0.ffn_down_t.weight"].offset)


def timed_loop(fn, seconds, max_n):
    n, t0 = 0, time.perf_counter()
    while True:
        fn(n)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= max_n:
            return n, el


def cpu_baseline_sparse(args, up, dn, wup, wout, X, thrs):
    """The oracle's restatement of ffnFlash path 2 (predictor.go:51-83 +
    ffn_flash.go:254-299) on a bounded sample of tokens.  Reported: the
    reference's own arrangement, rows read from a page-cached GGUF file by a
    32-thread pread pool that dequantizes them (ReadRowsParallel,
    storage.go:246-319) and the arithmetic on one thread; alongside it, the
    same arithmetic on rows already in memory, one thread."""
    from oracle import refcpu as R

    path, off_up, off_dn = layer_file(up, dn, R.Q4_0)
    try:
        log("cpu baseline: oracle predict + ffnSparseLoad, 32-thread pread pool")

        def faithful(i):
            x = X[i % X.shape[0]]
            active, _ = R.predict(wup, wout, None, x, float(thrs[i % X.shape[0]]))
            R.ffn_sparse_load_file(path, off_up, off_dn, R.Q4_0, H, FF, x, active, nthreads=32)

        n, el = timed_loop(faithful, args.cpu_seconds, args.cpu_max_tokens)
    finally:
        os.unlink(path)
    log("cpu baseline: the same on rows in memory, 1 thread")

    def in_memory(i):
        x = X[i % X.shape[0]]
        active, _ = R.predict(wup, wout, None, x, float(thrs[i % X.shape[0]]))
        R.ffn_sparse_load(up, dn, R.Q4_0, H, FF, x, active)

    n2, el2 = timed_loop(in_memory, args.cpu_seconds / 3, args.cpu_max_tokens)
    return {"value": n / el, "unit": "tokens/s", "cores": usable_cpus(), "kind": "port",
            "threads": "32 row-read threads (pread + dequant) and 1 arithmetic thread",
            **host_cpu(), "compute_only": n2 / el2,
            "sample": f"{n} decode tokens of the same layer (predict + sparse FFN), {el:.1f} s: "
                      f"up/down rows read from a page-cached GGUF file by a 32-thread pread pool "
                      f"with per-row dequant (ReadRowsParallel), arithmetic on 1 thread; rows in "
                      f"memory on 1 thread: {n2 / el2:.1f} tokens/s ({n2} tokens)"}


def bench_dense(args, torch, llg, dev, t):
    gg = llg.gguf
    L = args.layers
    g = torch.Generator(device="cuda")
    g.manual_seed(0x11A3A001)
    up = gg.quantize(torch.randn((FF, H), generator=g, device="cuda") * 0.02, t)
    down = gg.quantize(torch.randn((H, FF), generator=g, device="cuda") * 0.02, t)
    torch.cuda.synchronize()
    ups = [dev.upload_matrix(up, t, FF, H) for _ in range(L)]
    downs = [dev.upload_matrix(down, t, H, FF) for _ in range(L)]
    X = torch.randn((64, H), generator=g, device="cuda")
    out = torch.empty((64, H), device="cuda")
    torch.cuda.synchronize()
    tm = Timer(torch, dev.stream)

    def step(i):
        rc = dev.lib.llg_hipd_ffn_dense(dev.h, ups[i % L].id, downs[i % L].id, vp(X[i % 64]),
                                        gg.ACT_RELU, vp(out[i % 64]))
        if rc:
            dev.check(rc, "ffn_dense")

    for i in range(args.warmup):
        step(i)
    dev.sync()
    e0 = tm.event()
    for i in range(args.steps):
        step(i)
    e1 = tm.event()
    dev.sync()
    ms = e0.elapsed_time(e1) / args.steps
    alg = 2 * FF * gg.byte_size(t, H)
    gbs = alg / (ms * 1e-3) / 1e9
    for h_ in ups + downs:
        h_.release()
    return {"metric": "dense-FFN decode tokens/s + achieved HBM GB/s", "value": 1000.0 / ms,
            "unit": "tokens/s", "ms_per_step": ms, "dtype": "f32",
            "config": {"workload": f"falcon7b-ffn-layer-{gg.TYPE_NAMES[t].lower()}-dense-decode",
                       "d_model": H, "d_ff": FF, "layer_copies_rotated": L},
            "roofline": {"bound": "hbm", "kernel": "k_matvec_q (up) + k_matvec_q (down)",
                         "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None,
                         "alg_bytes_per_launch": alg, "avg_launch_us": ms * 1e3}}


SW_H, SW_FF = 4096, 11008  # LLaMA-7B layer (the SiLU architecture's dense FFN)


def bench_swiglu(args, torch, llg, dev, t):
    """One decode token through ffnSwiGLU (forward.go:368-389) at a LLaMA-7B
    layer's shape: gate and up matvecs fused (silu(g) * u), then down."""
    gg = llg.gguf
    L = args.layers
    g = torch.Generator(device="cuda")
    g.manual_seed(0x11A3A006)
    gate = gg.quantize(torch.randn((SW_FF, SW_H), generator=g, device="cuda") * 0.02, t)
    up = gg.quantize(torch.randn((SW_FF, SW_H), generator=g, device="cuda") * 0.02, t)
    down = gg.quantize(torch.randn((SW_H, SW_FF), generator=g, device="cuda") * 0.02, t)
    torch.cuda.synchronize()
    gates = [dev.upload_matrix(gate, t, SW_FF, SW_H) for _ in range(L)]
    ups = [dev.upload_matrix(up, t, SW_FF, SW_H) for _ in range(L)]
    downs = [dev.upload_matrix(down, t, SW_H, SW_FF) for _ in range(L)]
    X = torch.randn((64, SW_H), generator=g, device="cuda")
    out = torch.empty((64, SW_H), device="cuda")
    torch.cuda.synchronize()
    tm = Timer(torch, dev.stream)

    def step(i):
        rc = dev.lib.llg_hipd_ffn_swiglu(dev.h, gates[i % L].id, ups[i % L].id, downs[i % L].id,
                                         vp(X[i % 64]), vp(out[i % 64]))
        if rc:
            dev.check(rc, "ffn_swiglu")

    for i in range(args.warmup):
        step(i)
    dev.sync()
    e0 = tm.event()
    for i in range(args.steps):
        step(i)
    e1 = tm.event()
    dev.sync()
    ms = e0.elapsed_time(e1) / args.steps
    alg = 3 * SW_FF * gg.byte_size(t, SW_H)
    gbs = alg / (ms * 1e-3) / 1e9
    for h_ in gates + ups + downs:
        h_.release()
    return {"metric": "dense SwiGLU FFN decode tokens/s + achieved HBM GB/s", "value": 1000.0 / ms,
            "unit": "tokens/s", "ms_per_step": ms, "dtype": "f32",
            "config": {"workload": f"llama7b-ffn-layer-{gg.TYPE_NAMES[t].lower()}-swiglu-decode",
                       "d_model": SW_H, "d_ff": SW_FF, "layer_copies_rotated": L},
            "roofline": {"bound": "hbm",
                         "kernel": "k_matvec_q gated (gate+up, silu*mul) + k_matvec_q (down)",
                         "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None,
                         "alg_bytes_per_launch": alg, "avg_launch_us": ms * 1e3}}


WIN_K, WIN_SEQ, WIN_KEEP = 5, 64, 0.7


def window_sets(seed: int, n_tok: int) -> list:
    """Active sets of a decode sequence: 909 of 18176 neurons per token, 636
    drawn from the previous token's set and 273 uniform over the neurons not
    in it, each set ascending."""
    r = np.random.default_rng(seed)
    sets = [np.sort(r.choice(FF, N_ACTIVE, replace=False))]
    keep = int(round(WIN_KEEP * N_ACTIVE))
    for _ in range(n_tok - 1):
        kept = r.choice(sets[-1], keep, replace=False)
        rest = np.setdiff1d(np.arange(FF), sets[-1], assume_unique=True)
        new = r.choice(rest, N_ACTIVE - keep, replace=False)
        sets.append(np.sort(np.concatenate([kept, new])))
    return [s.astype(np.int32) for s in sets]


def window_loads(sets: list, k: int) -> list:
    """Neurons each Update must load: active minus the union of the last k
    sets (the resident set; inference/window.go:71-117)."""
    loads, ring = [], []
    for s in sets:
        res = set().union(*ring) if ring else set()
        loads.append(len(set(s.tolist()) - res))
        ring = (ring + [set(s.tolist())])[-k:]
    return loads


def bench_window(args, torch, llg, dev):
    """Sliding-window decode (window.go Update + FFNForward) over 64-token
    sequences of the Falcon-7B-shaped Q4_0 layer, k=5: per token the window
    state update, the gather of newly needed bundles into resident slots, and
    the gathered FFN over the resident rows (llg_hipd_window_step).  Sequence
    r runs on its own window over its own bundle copy."""
    gg = llg.gguf
    n_seq = (args.steps + WIN_SEQ - 1) // WIN_SEQ
    n_warm = max(1, (args.warmup + WIN_SEQ - 1) // WIN_SEQ)
    n_copies = min(args.layers, n_seq + n_warm)
    g = torch.Generator(device="cuda")
    g.manual_seed(0x11A3A002)
    up = gg.quantize(torch.randn((FF, H), generator=g, device="cuda") * 0.02, gg.Q4_0)
    dn = gg.quantize(torch.randn((FF, H), generator=g, device="cuda") * 0.02, gg.Q4_0)
    X = torch.randn((WIN_SEQ, H), generator=g, device="cuda")
    torch.cuda.synchronize()
    bundles = [dev.upload_bundle(up, dn, gg.Q4_0, H, FF) for _ in range(n_copies)]
    sets = window_sets(0x5E7, WIN_SEQ)
    loads = window_loads(sets, WIN_K)
    act = torch.tensor(np.stack(sets), device="cuda")
    nact = torch.full((WIN_SEQ, 1), N_ACTIVE, dtype=torch.int32, device="cuda")
    out = torch.empty((WIN_SEQ, H), device="cuda")
    wins = [llg.NeuronCache(dev, bundles[i % n_copies], WIN_K) for i in range(n_warm + n_seq)]
    lib = dev.lib

    def step(i):
        w, t = wins[i // WIN_SEQ], i % WIN_SEQ
        rc = lib.llg_hipd_window_step(dev.h, w.win.id, vp(X[t]), vp(act[t]), vp(nact[t]),
                                      gg.ACT_RELU, vp(out[t]))
        if rc:
            dev.check(rc, "window_step")

    tm = Timer(torch, dev.stream)
    for i in range(n_warm * WIN_SEQ):
        step(i)
    dev.sync()
    base = n_warm * WIN_SEQ
    e0 = tm.event()
    for i in range(args.steps):
        step(base + i)
    e1 = tm.event()
    dev.sync()
    ms = e0.elapsed_time(e1) / args.steps
    for w in wins:
        w.win.release()
    for b in bundles:
        b.release()
    n_load = float(np.mean([loads[i % WIN_SEQ] for i in range(args.steps)]))
    alg = N_ACTIVE * BUNDLE_ALG + 2 * n_load * BUNDLE_ALG
    gbs = alg / (ms * 1e-3) / 1e9
    res = {"metric": "sliding-window sparse-FFN decode tokens/s", "value": 1000.0 / ms,
           "unit": "tokens/s", "ms_per_step": ms, "dtype": "f32",
           "config": {"workload": "falcon7b-ffn-layer-q4_0-window5-decode64", "d_model": H,
                      "d_ff": FF, "window_k": WIN_K, "active": N_ACTIVE, "keep_from_prev": WIN_KEEP,
                      "tokens_per_sequence": WIN_SEQ, "mean_loaded_per_token": n_load,
                      "bundle_copies": n_copies},
           "roofline": {"bound": "hbm", "kernel": "k_win_step (up rows with the gather of "
                        "loaded bundles, down products, and the window update), one token",
                        "achieved": gbs, "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS, "traffic": None,
                        "alg_bytes_per_step": alg, "avg_step_us": ms * 1e3}}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline_window(args, up.cpu().numpy(), dn.cpu().numpy(),
                                                  X.cpu().numpy(), sets)
    return res


def cpu_baseline_window(args, up, dn, X, sets):
    """The oracle's NeuronCache (window.go Update + FFNForward) over the 64-token
    sequence, repeated on fresh caches up to the time bound.  Reported: new
    rows loaded from a page-cached GGUF file by the 32-thread pread pool
    (loadRows, window.go:208-216); alongside it, rows copied from memory."""
    from oracle import refcpu as R

    def run(make, seconds):
        n, t0 = 0, time.perf_counter()
        while True:
            nc = make()
            for t in range(WIN_SEQ):
                nc.update(sets[t])
                nc.ffn_forward(X[t], sets[t])
                n += 1
                if time.perf_counter() - t0 >= seconds:
                    break
            el = time.perf_counter() - t0
            if el >= seconds or n >= args.cpu_max_tokens:
                return n, el

    path, off_up, off_dn = layer_file(up, dn, R.Q4_0)
    try:
        log("cpu baseline: oracle window update + FFNForward, 32-thread pread pool")
        n, el = run(lambda: R.NeuronCache.from_file(FF, H, WIN_K, FF, path, off_up, off_dn,
                                                    R.Q4_0), args.cpu_seconds)
    finally:
        os.unlink(path)
    log("cpu baseline: the same with rows in memory, 1 thread")
    n2, el2 = run(lambda: R.NeuronCache(FF, H, WIN_K, FF, up, dn, R.Q4_0), args.cpu_seconds / 3)
    return {"value": n / el, "unit": "tokens/s", "cores": usable_cpus(), "kind": "port",
            "threads": "32 row-read threads (pread + dequant) and 1 arithmetic thread",
            **host_cpu(), "compute_only": n2 / el2,
            "sample": f"{n} window decode tokens (Update + FFNForward, k={WIN_K}), {el:.1f} s: "
                      f"new rows read from a page-cached GGUF file by a 32-thread pread pool "
                      f"(loadRows), arithmetic on 1 thread; rows in memory on 1 thread: "
                      f"{n2 / el2:.1f} tokens/s ({n2} tokens)"}


F4 = dict(n_layers=32, hidden=H, n_heads=71, n_kv=1, head_dim=64, ff=FF, vocab=65024,
          max_seq=2048, rank=RANK, rope_base=10000.0, eps=1e-5)
F4_PROMPT = 512


def falcon_weights(torch, gg, d, seed):
    """Random-init Falcon-7B-architecture weights, generated on the GPU:
    matrices N(0, 0.02) quantized to Q4_0, LayerNorm weight 1 and bias 0,
    predictors N(0, 0.05) in f32."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    h, L = d["hidden"], d["n_layers"]

    def q(r, c):
        return gg.quantize(torch.randn((r, c), generator=g, device="cuda") * 0.02, gg.Q4_0)

    def f(r, c, std):
        return (torch.randn((r, c), generator=g, device="cuda") * std).contiguous()

    w = {"embed": q(d["vocab"], h), "lm_head": q(d["vocab"], h),
         "out_w": np.ones(h, np.float32), "out_b": np.zeros(h, np.float32)}
    for k in ["norm_w", "norm_b", "wq", "wk", "wv", "wo", "pwup", "pwout", "up", "down_t"]:
        w[k] = []
    kvd, qd = d["n_kv"] * d["head_dim"], d["n_heads"] * d["head_dim"]
    for _ in range(L):
        w["norm_w"].append(np.ones(h, np.float32))
        w["norm_b"].append(np.zeros(h, np.float32))
        w["wq"].append(q(qd, h))
        w["wk"].append(q(kvd, h))
        w["wv"].append(q(kvd, h))
        w["wo"].append(q(h, qd))
        w["pwup"].append(f(d["rank"], h, 0.05))
        w["pwout"].append(f(d["ff"], d["rank"], 0.05))
        w["up"].append(q(d["ff"], h))
        w["down_t"].append(q(d["ff"], h))
    return w


def calibrate_thresholds(model, d, n_tok: int, frac: float, seed: int, rounds: int = 3):
    """Per-layer thresholds giving a mean active fraction `frac`: each round runs
    n_tok tokens from position 0 and sets every layer's threshold to the
    (1 - frac) quantile of its predictor logits (the thresholds of earlier
    layers change the inputs of later ones, hence the rounds)."""
    r = np.random.default_rng(seed)
    toks = r.integers(0, d["vocab"], n_tok)
    thr = np.full(d["n_layers"], np.float32(3.0e38))
    for _ in range(rounds):
        model.set_thresholds(thr)
        lgs = []
        for s, t in enumerate(toks):
            lgs.append(model.forward(int(t), s, pred_logits=True)[3])
        lg = np.stack(lgs)  # [n_tok, L, ff]
        thr = np.array([np.quantile(lg[:, l, :], 1.0 - frac) for l in range(d["n_layers"])],
                       np.float32)
    model.set_thresholds(thr)
    return thr


def bench_falcon(args, torch, llg, dev):
    """Full Falcon-7B-architecture decode (32 layers, 71 heads x 64 with one KV
    head, LayerNorm, NeoX RoPE, per-layer rank-128 predictor at 5%, sparse
    Q4_0 FFN, LM head over 65024): a 512-token random-id prompt (sequential
    prefill, as the reference runs it) then greedy decode chained on the
    device; one step = one generated token through the whole model."""
    gg = llg.gguf
    d = dict(F4)
    n_gen = max(1, min(args.steps, d["max_seq"] - F4_PROMPT))
    log("falcon: generating weights on the GPU (32 layers, Q4_0)")
    w = falcon_weights(torch, gg, d, 0x11A3A004)
    torch.cuda.synchronize()
    model = llg.FalconModel(dev, d, w, np.zeros(d["n_layers"], np.float32))
    thr = calibrate_thresholds(model, d, 16, 0.05, 0xCA1)
    r = np.random.default_rng(0x9707)
    prompt = r.integers(0, d["vocab"], F4_PROMPT).astype(np.int32)
    toks = torch.tensor(prompt, device="cuda")
    gen = torch.zeros(n_gen + 2, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    tm = Timer(torch, dev.stream)
    p0 = tm.event()
    for s in range(F4_PROMPT):
        out = gen.data_ptr() if s == F4_PROMPT - 1 else gen.data_ptr() + 4 * (n_gen + 1)
        model.step_device(toks.data_ptr() + 4 * s, s, out)
    p1 = tm.event()
    for i in range(n_gen):
        model.step_device(gen.data_ptr() + 4 * i, F4_PROMPT + i, gen.data_ptr() + 4 * (i + 1))
    p2 = tm.event()
    dev.sync()
    prefill_ms = p0.elapsed_time(p1)
    ms = p1.elapsed_time(p2) / n_gen
    # active neurons per layer on one more token (host path)
    _, _, na = model.forward(int(gen[n_gen].item()), F4_PROMPT + n_gen - 1)
    mean_act = float(na.mean())
    hd, kvd = d["head_dim"], d["n_kv"] * d["head_dim"]
    row = gg.byte_size(gg.Q4_0, d["hidden"])
    mean_pos = F4_PROMPT + n_gen / 2.0
    per_layer = ((d["n_heads"] * hd + 2 * kvd) * row + d["hidden"] * gg.byte_size(
        gg.Q4_0, d["n_heads"] * hd) + PRED_BYTES + mean_act * BUNDLE_ALG +
        2 * kvd * 4 * mean_pos + 2 * d["hidden"] * 4 * 2)
    alg = d["n_layers"] * per_layer + d["vocab"] * row + row
    gbs = alg / (ms * 1e-3) / 1e9
    res = {"metric": "full-model decode tokens/s", "value": 1000.0 / ms, "unit": "tokens/s",
           "ms_per_step": ms, "dtype": "f32",
           "config": {"workload": "falcon7b-arch-32layer-q4_0-5pct-sparse-greedy-decode",
                      "n_layers": 32, "d_model": d["hidden"], "heads": "71 x 64, 1 KV head",
                      "d_ff": d["ff"], "vocab": d["vocab"], "kv_len": d["max_seq"],
                      "prompt_tokens": F4_PROMPT, "generated_tokens": n_gen,
                      "prefill_ms": prefill_ms, "prefill_tokens_per_s": F4_PROMPT / prefill_ms * 1e3,
                      "mean_active_per_layer": mean_act},
           "roofline": {"bound": "hbm", "kernel": "one decode token: k_embed, 32 x (k_matvec_q "
                        "qkv with the LayerNorm prologue, k_attn with the predictor products, "
                        "k_tile_wo_ffn (the predictor's hidden units, the tiles, then wo with the "
                        "attention merge), k_tile_reduce) + "
                        "k_out_norm, k_matvec_q lm head, k_argmax",
                        "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": gbs / HBM_PEAK_GBS, "traffic": None, "alg_bytes_per_step": alg,
                        "avg_step_us": ms * 1e3}}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline_falcon(args, d, w, thr, prompt)
    model.release()
    return res


def falcon_ffn_file(d, hw, t):
    """Every layer's ffn_up and transposed ffn_down (GGUF dims [hidden, ff], one
    row per neuron) in one GGUF file in the temp directory, read once so that it
    sits in the page cache as the reference's weights do after the first token.
    Returns (path, up offsets, down offsets)."""
    import tempfile

    from llg import gguf_file as GF

    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    L, h, ff = d["n_layers"], d["hidden"], d["ff"]
    tensors = []
    for l in range(L):
        tensors += [(f"blk.{l}.ffn_up.weight", [h, ff], t, hw["up"][l]),
                    (f"blk.{l}.ffn_down_t.weight", [h, ff], t, hw["down_t"][l])]
    GF.write_gguf(path, [("general.architecture", GF.T_STRING, "falcon")], tensors)
    with open(path, "rb") as f:
        while f.read(1 << 24):
            pass
    gf = GF.open_gguf(path)
    return (path, [gf.by_name[f"blk.{l}.ffn_up.weight"].offset for l in range(L)],
            [gf.by_name[f"blk.{l}.ffn_down_t.weight"].offset for l in range(L)])


def cpu_baseline_falcon(args, d, w, thr, prompt):
    """The oracle's ForwardFlash in the reference's arrangement, timed on
    positions inside the GPU's timed range: the 512-token prompt runs first,
    untimed, with the oracle's rows split over every usable CPU (the same
    results bit for bit); then greedy decode from position 512 is timed on one
    arithmetic thread with each layer's FFN rows read from a page-cached GGUF
    file by the 32-thread pread pool (ffn_flash.go:262-270, ReadRowsParallel
    storage.go:246-319), the attention, embedding and LM head dequantized to
    fp32 at load as the reference does."""
    from oracle import refcpu as R

    def host(a):
        return a.cpu().numpy() if hasattr(a, "is_cuda") else np.asarray(a)

    hw = {k: ([host(x) for x in v] if isinstance(v, list) else host(v)) for k, v in w.items()}
    ncpu = usable_cpus()
    log("cpu baseline: writing the 32 layers' FFN rows to a GGUF file")
    path, up_off, dn_off = falcon_ffn_file(d, hw, R.Q4_0)
    try:
        ref = R.Falcon(d, hw, thr)
        log(f"cpu baseline: oracle prompt of {len(prompt)} tokens, untimed, {ncpu} threads")
        R.set_threads(ncpu)
        try:
            t0 = time.perf_counter()
            for s in range(len(prompt)):
                lg, _ = ref.forward(int(prompt[s]), s)
                if s % 128 == 127:
                    log(f"cpu baseline: prompt position {s} ({time.perf_counter() - t0:.0f} s)")
        finally:
            R.set_threads(1)
        log("cpu baseline: timed greedy decode, 1 arithmetic thread + 32-thread row reads")
        ref.ffn_file(path, up_off, dn_off, nthreads=32)
        pos, n = len(prompt), 0
        nxt = R.argmax(lg)
        t0 = time.perf_counter()
        while pos < d["max_seq"]:
            lg, _ = ref.forward(nxt, pos)
            nxt = R.argmax(lg)
            pos += 1
            n += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds:
                break
    finally:
        os.unlink(path)
    return {"value": n / el, "unit": "tokens/s", "cores": ncpu, "kind": "port",
            "threads": "1 arithmetic thread and a 32-thread FFN row-read pool (pread + dequant)",
            **host_cpu(),
            "sample": f"{n} greedy tokens at positions {len(prompt)}-{pos - 1} after the "
                      f"{len(prompt)}-token prompt (run first, untimed, on {ncpu} threads), "
                      f"{el:.1f} s: FFN rows read per token from a page-cached GGUF file by "
                      f"the 32-thread pread pool, attention/embedding/LM head dequantized to "
                      f"fp32 at load, weights in host memory"}


MOE_D, MOE_FF, MOE_E, MOE_K, MOE_PREFILL = 4096, 14336, 8, 2, 512
MFMA_F16_PEAK_TFLOPS = 2500.0


def bench_moe(args, torch, llg, dev, prefill: bool):
    """Mixtral-shaped MoE layer (d=4096, 8 SwiGLU experts of 14336, top-2, Q4_0).
    decode: one token per step (router + 2 experts' gate/up/down matvecs +
    combine), x fresh per step.  prefill: 512 tokens per step, grouped per
    expert into MFMA GEMMs."""
    gg = llg.gguf
    L = args.layers
    g = torch.Generator(device="cuda")
    g.manual_seed(0x30E00003)
    router = torch.randn((MOE_E, MOE_D), generator=g, device="cuda") * 0.02
    mats = []
    for rows, cols in [(MOE_E * MOE_FF, MOE_D)] * 2 + [(MOE_E * MOE_D, MOE_FF)]:
        q = gg.quantize(torch.randn((rows, cols), generator=g, device="cuda") * 0.02, gg.Q4_0)
        mats.append([dev.upload_matrix(q, gg.Q4_0, rows, cols) for _ in range(L)])
        del q
    rh = dev.upload_matrix(router, gg.F32, MOE_E, MOE_D)
    n_tok = MOE_PREFILL if prefill else 1
    nx = 4 if prefill else 64
    X = torch.randn((nx, n_tok, MOE_D), generator=g, device="cuda")
    out = torch.empty((n_tok, MOE_D), device="cuda")
    ids = torch.empty((n_tok, MOE_K), dtype=torch.int32, device="cuda")
    w = torch.empty((n_tok, MOE_K), device="cuda")
    torch.cuda.synchronize()
    tm = Timer(torch, dev.stream)

    def step(i):
        l = i % L
        rc = dev.lib.llg_hipd_moe_ffn(dev.h, rh.id, mats[0][l].id, mats[1][l].id, mats[2][l].id,
                                      MOE_E, MOE_K, vp(X[i % nx]), n_tok, vp(out), vp(ids), vp(w))
        if rc:
            dev.check(rc, "moe_ffn")

    for i in range(args.warmup):
        step(i)
    dev.sync()
    e0 = tm.event()
    for i in range(args.steps):
        step(i)
    e1 = tm.event()
    dev.sync()
    ms = e0.elapsed_time(e1) / args.steps
    q4 = gg.byte_size(gg.Q4_0, MOE_D)          # per row of gate/up; down rows are eff wide
    expert_bytes = 2 * MOE_FF * q4 + MOE_D * gg.byte_size(gg.Q4_0, MOE_FF)
    hit = int(torch.unique(ids).numel())
    for ms_ in mats:
        for h_ in ms_:
            h_.release()
    rh.release()
    if prefill:
        flops = n_tok * MOE_K * 3 * 2 * MOE_D * MOE_FF
        tf = flops / (ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "kernel": "k_moe_gemm<0> (gate/up+SwiGLU) + k_moe_gemm<1> (down) "
                "+ grouping/convert/combine (one 512-token step)",
                "achieved": tf, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": tf / MFMA_F16_PEAK_TFLOPS, "traffic": None,
                "alg_flops_per_step": flops, "alg_weight_bytes_per_step": hit * expert_bytes,
                "avg_step_us": ms * 1e3}
        wl = "mixtral-moe-layer-q4_0-top2-prefill512"
        dtype = "f16 x q4_0 -> f32"
    else:
        alg = MOE_K * expert_bytes
        gbs = alg / (ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": "k_moe_router + k_moe_gateup + k_moe_down (one token)",
                "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": gbs / HBM_PEAK_GBS, "traffic": None, "alg_bytes_per_step": alg,
                "avg_step_us": ms * 1e3}
        wl = "mixtral-moe-layer-q4_0-top2-decode"
        dtype = "f32"
    return {"metric": "MoE FFN tokens/s", "value": n_tok * 1000.0 / ms, "unit": "tokens/s",
            "ms_per_step": ms, "dtype": dtype,
            "config": {"workload": wl, "d_model": MOE_D, "expert_ff": MOE_FF, "n_experts": MOE_E,
                       "top_k": MOE_K, "tokens_per_step": n_tok, "layer_copies_rotated": L},
            "roofline": roof}


def default_layers(workload: str) -> int:
    """Distinct HBM copies a workload rotates over (enough to defeat the MALL)."""
    return {"sparse": 128, "all": 128, "window": 16, "moe-decode": 8,
            "moe-prefill": 1}.get(workload, 6)


def set_vs_baseline(res: dict) -> None:
    """The reference publishes no figure for these metrics; its baseline is its
    own CPU path timed in this run on this host (cpu_baseline), so vs_baseline
    is the ratio to that, and null when the CPU leg was skipped."""
    cb = res.get("cpu_baseline")
    res["vs_baseline"] = res["value"] / cb["value"] if cb and cb.get("value") else None
    res["vs_baseline_basis"] = ("value / cpu_baseline.value (the reference CPU path timed in "
                                "this run; no published figure exists)" if cb else None)


def run_workload(args, torch, llg, dev) -> dict:
    gg = llg.gguf
    if args.workload == "sparse":
        return bench_sparse(args, torch, llg, dev)
    if args.workload == "window":
        return bench_window(args, torch, llg, dev)
    if args.workload == "falcon-decode":
        return bench_falcon(args, torch, llg, dev)
    if args.workload.startswith("moe-"):
        return bench_moe(args, torch, llg, dev, args.workload == "moe-prefill")
    if args.workload.startswith("swiglu-"):
        t = {"swiglu-q4_0": gg.Q4_0, "swiglu-q8_0": gg.Q8_0, "swiglu-f16": gg.F16}[args.workload]
        return bench_swiglu(args, torch, llg, dev, t)
    t = {"dense-q4_0": gg.Q4_0, "dense-q8_0": gg.Q8_0, "dense-f16": gg.F16}[args.workload]
    return bench_dense(args, torch, llg, dev, t)


# The other workloads of the default run: (name, steps, warmup, CPU baseline).
# Config 1 (dense, three types), config 2 (window), config 3 (MoE decode and
# 512-token prefill), config 4 (the 32-layer model, 256 greedy tokens after the
# 512-token prompt, its CPU baseline at positions from 512) and the SwiGLU
# dense FFN at a LLaMA-7B layer.
SECONDARY = [("dense-q4_0", 500, 50, False), ("dense-q8_0", 500, 50, False),
             ("dense-f16", 500, 50, False), ("window", 640, 64, True),
             ("moe-decode", 500, 50, False), ("moe-prefill", 40, 5, False),
             ("falcon-decode", 256, 0, True), ("swiglu-q4_0", 500, 50, False),
             ("swiglu-q8_0", 500, 50, False), ("swiglu-f16", 500, 50, False)]


def run_secondary(args, torch, llg, dev) -> dict:
    """Each other workload in turn, in this process, each with its own result
    (or the error it raised, so that one failing workload does not lose the
    others)."""
    import gc

    out = {}
    for name, steps, warmup, cpu in SECONDARY:
        a = argparse.Namespace(**vars(args))
        a.workload, a.steps, a.warmup = name, steps, warmup
        a.layers = default_layers(name)
        a.no_cpu = args.no_cpu or not cpu
        a.cpu_seconds = min(args.cpu_seconds, 15.0)
        log(f"workload {name}: {steps} steps")
        t0 = time.perf_counter()
        try:
            r = run_workload(a, torch, llg, dev)
            r.update({"steps": steps, "warmup": warmup})
            r.setdefault("cpu_baseline", None)
            set_vs_baseline(r)
        except Exception as e:  # a host-side error of one workload
            r = {"error": f"{type(e).__name__}: {e}"}
            log(f"workload {name} failed: {r['error']}")
        r["wall_s"] = time.perf_counter() - t0
        out[name] = r
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="all",
                    choices=["all", "sparse", "dense-q4_0", "dense-q8_0", "dense-f16", "window",
                             "moe-decode", "moe-prefill", "falcon-decode", "swiglu-q4_0",
                             "swiglu-q8_0", "swiglu-f16"],
                    help="all (default): the sparse step as the headline line, then every "
                         "other workload in the same process under its `workloads` key")
    ap.add_argument("--layers", type=int, default=0,
                    help="distinct HBM copies rotated per step (0 = enough to defeat the MALL)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-max-tokens", type=int, default=2000)
    ap.add_argument("--calib-mib", type=int, default=0,
                    help="first run 4 streaming copies of this many MiB (torch elementwise "
                         "kernel reading and writing the size each), the known-size reference "
                         "for rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the sparse-FFN path is measured on a single MI355X; a sharded layer would "
              "split the neurons across GPUs and all-reduce the 18 KB output per layer)",
              file=sys.stderr)
        sys.exit(2)
    if args.layers <= 0:
        args.layers = default_layers(args.workload)

    import torch
    import llg

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = llg.Device()
    gg = llg.gguf
    if args.calib_mib > 0:
        n = args.calib_mib * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty(n, device="cuda")
        for _ in range(4):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log(f"calibration: 4 copies of {args.calib_mib} MiB (read and write each)")
        del src, dst
    if args.workload == "all":
        res = bench_sparse(args, torch, llg, dev)
        res["workloads"] = run_secondary(args, torch, llg, dev)
    else:
        res = run_workload(args, torch, llg, dev)
    res.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                "higher_is_better": True, "scaling": "weak",
                "data": "synthetic (seeded N(0,0.02) weights, N(0,1) inputs)"})
    res.setdefault("cpu_baseline", None)
    set_vs_baseline(res)
    order = ["metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
             "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config", "roofline",
             "cpu_baseline"]
    line = {k: res[k] for k in order if k in res}
    line.update({k: v for k, v in res.items() if k not in line})
    dev.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
