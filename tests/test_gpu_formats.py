"""GPU: models and bundles loaded from files (GGUF through the loader, BNDL
bundle files) against the oracle on the weights the files were written from,
and the no-RoPE model against the oracle.

The file side is this build's reader, loader and bundle writer (gguf/reader.go:
27-115, model/loader.go:102-242, flash/bundle.go:37-216); the oracle side is
refcpu on the original in-memory weights, or reading the rows from the GGUF
file itself as ReadRowsParallel does (flash/storage.go:246-319)."""
import numpy as np
import pytest

import llg
import llg.bundle as B
import llg.gguf as gg
import llg.gguf_file as G
import llg.loader as LD
from oracle import refcpu as R
from tests.helpers import make_falcon, make_sparse_layer, max_rel_err, normal, ref_falcon_f64

pytestmark = pytest.mark.gpu

TOL = 1e-3
FALCON = dict(n_layers=2, hidden=256, n_heads=4, n_kv=1, head_dim=64, ff=512, vocab=300,
              max_seq=32, rank=16, rope_base=10000.0, eps=1e-5)


def _decode_vs_oracle(m, ref, toks):
    """The file-loaded device model against the oracle token by token: active
    counts exact (thresholds sit in wide logit gaps), logits within the FFN
    bar, the greedy token equal where the top-2 gap is clear."""
    for s, tk in enumerate(toks):
        lg, nxt, na = m.forward(int(tk), s)
        rl, rn = ref.forward(int(tk), s)
        assert np.array_equal(na, rn), (s, na, rn)
        assert max_rel_err(lg, rl) <= TOL, s
        srt = np.sort(rl)
        if srt[-1] - srt[-2] > 1e-3 * np.max(np.abs(rl)):
            assert nxt == R.argmax(rl), s


@pytest.mark.parametrize("act", [gg.ACT_RELU, None])
def test_load_falcon_matches_oracle(dev, rng, tmp_path, act):
    """Predictors and thresholds read from the file; act None takes the
    architecture's activation (GELU for falcon, loader.go:56)."""
    d = dict(FALCON)
    w = make_falcon(rng, d)
    toks = rng.integers(0, d["vocab"], 6)
    _, _, thr = ref_falcon_f64(w, d, toks)
    p = tmp_path / "falcon.gguf"
    LD.write_falcon_gguf(p, d, w, gg.Q4_0, thresholds=thr)
    m, hp = LD.load_falcon(dev, p, act=act)
    assert hp["n_layers"] == 2 and hp["head_dim"] == 64 and m.dims["max_seq"] == 32
    ref = R.Falcon(d, w, thr, act=gg.ACT_GELU if act is None else act)
    _decode_vs_oracle(m, ref, toks)
    m.release()


def test_load_falcon_tied_output_external_predictors(dev, rng, tmp_path):
    d = dict(FALCON)
    w = make_falcon(rng, d)
    w["lm_head"] = w["embed"]
    toks = rng.integers(0, d["vocab"], 5)
    _, _, thr = ref_falcon_f64(w, d, toks)
    p = tmp_path / "tied.gguf"
    LD.write_falcon_gguf(p, d, w, gg.Q4_0, with_predictors=False,
                         tie_output=True)
    assert "output.weight" not in G.open_gguf(p).by_name
    preds = list(zip(w["pwup"], w["pwout"]))
    m, _ = LD.load_falcon(dev, p, predictors=preds, thresholds=thr, act=gg.ACT_RELU, max_seq=20)
    ref = R.Falcon(dict(d, max_seq=20), w, thr)
    _decode_vs_oracle(m, ref, toks)
    m.release()


def test_falcon_without_rope(dev, rng):
    """rope_base 0: no rotation (forward.go:249-252), against the oracle."""
    d = dict(FALCON, rope_base=0.0)
    w = make_falcon(rng, d)
    toks = rng.integers(0, d["vocab"], 6)
    _, nact, thr = ref_falcon_f64(w, d, toks)
    ref = R.Falcon(d, w, thr)
    m = llg.FalconModel(dev, d, w, thr)
    for s, tk in enumerate(toks):
        lg, _, na = m.forward(int(tk), s)
        rl, rn = ref.forward(int(tk), s)
        assert np.array_equal(na, rn) and np.array_equal(na, nact[s])
        assert max_rel_err(lg, rl) <= TOL, s
    m.release()


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
def test_bundle_file_upload(dev, rng, tmp_path, t):
    """Bundles uploaded from files, typed (the row type in the reserved word)
    and the reference's float32 layout (bundle.go:66-111), against the oracle
    reading the same rows from the GGUF layer file (storage.go:246-319):
    dequantized rows bit-exact, and the gathered FFN within the bar for
    sorted, unsorted and repeated neuron lists."""
    h, ff = 256, 512
    up, dn = make_sparse_layer(rng, h, ff, t)
    p = tmp_path / "l.gguf"
    G.write_gguf(p, [], [("blk.0.ffn_up.weight", [h, ff], t, up),
                         ("blk.0.ffn_down.weight", [h, ff], t, dn)])
    f = G.open_gguf(p)
    ui, di = f.by_name["blk.0.ffn_up.weight"], f.by_name["blk.0.ffn_down.weight"]
    B.create_bundle(tmp_path / "q.bundle", f, ui, di, row_type=None)
    B.create_bundle(tmp_path / "f.bundle", f, ui, di)
    from_file = B.open_bundle(tmp_path / "q.bundle").upload(dev)
    f32 = B.open_bundle(tmp_path / "f.bundle").upload(dev)
    # rows as the oracle reads them from the GGUF file: [up_i | down_i] per neuron
    allr = np.arange(ff, dtype=np.int32)
    rows = np.concatenate([R.read_rows_file(p, ui.offset, t, h, ff, allr),
                           R.read_rows_file(p, di.offset, t, h, ff, allr)], axis=1)
    assert np.array_equal(dev.dequant(from_file, 0, ff).view(np.uint32), rows.view(np.uint32))
    assert np.array_equal(dev.dequant(f32, 0, ff).view(np.uint32), rows.view(np.uint32))
    x = normal(rng, h, 1.0)
    active = np.sort(rng.choice(ff, 60, replace=False)).astype(np.int32)
    lists = [active, active[::-1].copy(), np.concatenate([active, active[:7]])]
    for a in lists:
        ref = R.ffn_sparse_load_file(p, ui.offset, di.offset, t, h, ff, x, a)
        for b in (from_file, f32):
            assert max_rel_err(llg.ffn_sparse_load(dev, b, x, a), ref) <= TOL
    for b in (from_file, f32):
        b.release()
