"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

The reference (AndersHsueh/llama.go) has no tests, testdata or golden vectors
and cannot be compiled here (no Go toolchain), so these fixtures are written
by the oracle (oracle/refcpu.c) on seeded inputs.  They freeze its outputs:
tests/test_golden.py re-runs the oracle on the stored inputs and requires the
stored outputs bit for bit, and the GPU tests compare the HIP path with them.

Run:  python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "llama.go_amd"))

from oracle import refcpu as R  # noqa: E402
from tests.helpers import normal, quant, threshold_for, window_sets  # noqa: E402


def kat_blocks():
    """Hand-built Q4_0 / Q8_0 blocks and f16 specials with their decodes."""
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x3C00, 0xC000, 0x7BFF, 0x7C00, 0xFC00,
                         0x7E01, 0x7C01, 0xFE00, 0x3555, 0x0200], np.uint16)
    f16_out = np.array([R.f16_to_f32_bits(int(h)) for h in specials], np.uint32)
    q4 = []
    for dbits in (0x3C00, 0xB800, 0x0001, 0x4A00):
        qs = [(((2 * i + 1) % 16) << 4) | ((2 * i) % 16) for i in range(16)]
        q4.append([dbits & 0xFF, dbits >> 8] + qs)
    q4 = np.array(q4, np.uint8)
    q4_out = np.stack([R.dequantize(b, R.Q4_0) for b in q4])
    q8 = []
    for dbits, base in ((0x4000, -16), (0x3C00, -128), (0x2E66, 96)):
        qs = (np.arange(32) + base).astype(np.int8).view(np.uint8)
        q8.append(np.concatenate([[dbits & 0xFF, dbits >> 8], qs]).astype(np.uint8))
    q8 = np.array(q8, np.uint8)
    q8_out = np.stack([R.dequantize(b, R.Q8_0) for b in q8])
    np.savez(HERE / "dequant_kat.npz", f16_in=specials, f16_out_bits=f16_out, q4_in=q4,
             q4_out=q4_out, q8_in=q8, q8_out=q8_out)


def pred_tiny(rng):
    h, ff, rank = 64, 256, 16
    wup, wout = normal(rng, (rank, h), 0.05), normal(rng, (ff, rank), 0.05)
    bias, a = normal(rng, ff, 0.01), normal(rng, h, 1.0)
    _, lg = R.predict(wup, wout, bias, a, 0.0)
    thr = threshold_for(lg, 13)
    active, logits = R.predict(wup, wout, bias, a, thr)
    np.savez(HERE / "pred_tiny.npz", wup=wup, wout=wout, bias=bias, a=a,
             threshold=np.float32(thr), logits=logits, active=active)


def ffn_sparse_tiny(rng):
    h, ff = 64, 128
    data = {}
    x = normal(rng, h, 1.0)
    active = np.sort(rng.choice(ff, 20, replace=False)).astype(np.int32)
    data["x"], data["active"] = x, active
    for name, t in (("q4_0", R.Q4_0), ("q8_0", R.Q8_0), ("f16", R.F16)):
        up, dn = quant(normal(rng, (ff, h), 0.02), t), quant(normal(rng, (ff, h), 0.02), t)
        data[f"{name}_up"], data[f"{name}_down_t"] = up, dn
        for act_name, act in (("relu", R.ACT_RELU), ("silu", R.ACT_SILU), ("gelu", R.ACT_GELU)):
            data[f"{name}_out_{act_name}"] = R.ffn_sparse_load(up, dn, t, h, ff, x, active, act)
    np.savez(HERE / "ffn_sparse_tiny.npz", **data)


def ffn_dense_tiny(rng):
    h, ff = 64, 96
    up = quant(normal(rng, (ff, h), 0.02), R.Q4_0)
    down = quant(normal(rng, (h, ff), 0.02), R.Q4_0)
    x = normal(rng, h, 1.0)
    out = R.ffn_dense(up, down, R.Q4_0, h, ff, x)
    np.savez(HERE / "ffn_dense_tiny.npz", up=up, down=down, x=x, out=out)


def window_tiny(rng):
    h, ff, k, steps = 32, 64, 5, 16
    up, dn = quant(normal(rng, (ff, h), 0.02), R.Q4_0), quant(normal(rng, (ff, h), 0.02), R.Q4_0)
    sets = window_sets(rng, ff, 12, steps, 0.7)
    nc = R.NeuronCache(256, h, k, ff, up, dn, R.Q4_0)
    xs = normal(rng, (steps, h), 1.0)
    n_loaded, n_cached, outs, resident = [], [], [], np.zeros((steps, ff), np.uint8)
    for t, A in enumerate(sets):
        n_loaded.append(nc.update(A).size)
        n_cached.append(nc.num_cached())
        resident[t, nc.resident()] = 1
        outs.append(nc.ffn_forward(xs[t], A))
    np.savez(HERE / "window_tiny.npz", up=up, down_t=dn, k=np.int32(k),
             sets=np.stack(sets), xs=xs, n_loaded=np.array(n_loaded, np.int32),
             n_cached=np.array(n_cached, np.int32), resident=resident, outs=np.stack(outs))


def moe_tiny(rng):
    d, eff, E, k, n_tok = 64, 96, 4, 2, 16
    router = normal(rng, (E, d), 0.2)
    gate = quant(normal(rng, (E * eff, d), 0.05), R.Q4_0)
    up = quant(normal(rng, (E * eff, d), 0.05), R.Q4_0)
    down = quant(normal(rng, (E * d, eff), 0.05), R.Q4_0)
    x = normal(rng, (n_tok, d), 1.0)
    outs, ids, ws = [], [], []
    for t in range(n_tok):
        o, i, w = R.moe_ffn(router, gate, up, down, R.Q4_0, d, eff, E, k, x[t])
        outs.append(o)
        ids.append(i)
        ws.append(w)
    lg = normal(rng, (64, 8), 1.5)
    lg[0] = 0.0
    lg[1] = [0, 1, 1, 1, 0, 0, 0, 0]
    r_ids, r_w = zip(*[R.moe_route(lg[t], 2) for t in range(64)])
    np.savez(HERE / "moe_tiny.npz", router=router, gate=gate, up=up, down=down, x=x,
             k=np.int32(k), out=np.stack(outs), ids=np.stack(ids), w=np.stack(ws),
             route_logits=lg, route_ids=np.stack(r_ids), route_w=np.stack(r_w))


def ffn_swiglu_tiny(rng):
    """ffnSwiGLU (forward.go:368-389) on Q4_0, Q8_0 and F16 weights."""
    h, ff = 64, 160
    x = normal(rng, h, 1.0)
    data = {"x": x}
    g32, u32, d32 = (normal(rng, (ff, h), 0.1), normal(rng, (ff, h), 0.1),
                     normal(rng, (h, ff), 0.1))
    for name, t in (("q4_0", R.Q4_0), ("q8_0", R.Q8_0), ("f16", R.F16)):
        g, u, d = quant(g32, t), quant(u32, t), quant(d32, t)
        data.update({f"{name}_gate": g, f"{name}_up": u, f"{name}_down": d,
                     f"{name}_out": R.ffn_swiglu(g, u, d, t, h, ff, x)})
    np.savez(HERE / "ffn_swiglu_tiny.npz", **data)


def main():
    R.build()
    rng = np.random.default_rng(0x11A3A000)
    kat_blocks()
    pred_tiny(rng)
    ffn_sparse_tiny(rng)
    ffn_dense_tiny(rng)
    window_tiny(rng)
    moe_tiny(rng)
    ffn_swiglu_tiny(np.random.default_rng(0x11A3A005))  # own stream: earlier fixtures unchanged
    for p in sorted(HERE.glob("*.npz")):
        print(f"{p.name}: {p.stat().st_size} bytes")


if __name__ == "__main__":
    main()
