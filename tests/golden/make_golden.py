"""Write the committed golden fixtures for the gdn2 tests.

The reference repository ships no stored tensors (its tests are relative
checks only), so the fixtures are produced by this repository's float64
oracle (oracle/gdn2_oracle.py), itself pinned by closed forms, the
third-party scalar gated delta rule and finite differences in
tests/test_oracle.py.  Inputs are stored as float32 (exact in every kernel
dtype path that upcasts), outputs as float64.

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import gdn2_oracle as orc  # noqa: E402


def _inputs(B, T, H, K, V, seed, h0_std=0.1):
    rng = np.random.default_rng(seed)
    f = np.float32
    d = dict(
        q=rng.standard_normal((B, T, H, K)).astype(f),
        k=rng.standard_normal((B, T, H, K)).astype(f),
        v=rng.standard_normal((B, T, H, V)).astype(f),
        g=(-np.logaddexp(0.0, rng.standard_normal((B, T, H, K)) + 2.0)).astype(f),
        b=(1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H, K))))).astype(f),
        w=(1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H, V))))).astype(f),
    )
    d["h0"] = (rng.standard_normal((B, H, K, V)) * h0_std).astype(f)
    return d


def make_fwd():
    inp = _inputs(1, 100, 2, 32, 16, seed=2024)
    x = {n: a.astype(np.float64) for n, a in inp.items()}
    o, ht = orc.recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["b"], x["w"], x["h0"])
    np.savez_compressed(HERE / "gdn2_fwd_T100_H2_K32_V16.npz", **inp, o=o, ht=ht)


def make_varlen():
    inp = _inputs(1, 90, 2, 16, 16, seed=7)
    cu = np.array([0, 1, 40, 40, 90], dtype=np.int64)
    rng = np.random.default_rng(8)
    inp["h0"] = (rng.standard_normal((4, 2, 16, 16)) * 0.1).astype(np.float32)
    x = {n: a.astype(np.float64) for n, a in inp.items()}
    o, ht = orc.recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["b"], x["w"], x["h0"], cu_seqlens=cu)
    np.savez_compressed(HERE / "gdn2_varlen_T90_N4.npz", **inp, cu_seqlens=cu, o=o, ht=ht)


def make_bwd():
    inp = _inputs(1, 24, 2, 8, 8, seed=99)
    rng = np.random.default_rng(100)
    do = rng.standard_normal((1, 24, 2, 8)).astype(np.float32)
    dht = rng.standard_normal((1, 2, 8, 8)).astype(np.float32)
    x = {n: a.astype(np.float64) for n, a in inp.items()}
    dq, dk, dv, dg, db, dw, dh0 = orc.recurrent_vjp(
        x["q"], x["k"], x["v"], x["g"], x["b"], x["w"], do.astype(np.float64),
        dht.astype(np.float64), x["h0"])
    np.savez_compressed(HERE / "gdn2_bwd_T24_H2_K8_V8.npz", **inp, do=do, dht=dht, dq=dq, dk=dk,
                        dv=dv, dg=dg, db=db, dw=dw, dh0=dh0)


def make_config0():
    """BASELINE config 0 (B1 T512 H4 K=V=64, seed 0): input fingerprints + sampled outputs."""
    inp = orc.make_inputs(0, 1, 512, 4, 64, 64)
    o, ht = orc.recurrent_fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["b"], inp["w"])
    fp = np.array([float(np.sum(inp[n])) for n in ("q", "k", "v", "g", "b", "w")])
    np.savez_compressed(HERE / "gdn2_config0_fingerprint.npz", input_sums=fp,
                        o_head0_first64=o[0, :64, 0], o_norm=np.linalg.norm(o),
                        o_token_norms=np.linalg.norm(o[0], axis=(1, 2)), ht=ht)


if __name__ == "__main__":
    make_fwd()
    make_varlen()
    make_bwd()
    make_config0()
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)
