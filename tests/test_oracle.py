"""Pin the float64 oracle (CPU).

The reference ships no golden tensors, so every oracle function is checked
against something that does not restate its own formula:
  * closed forms (linear attention, single token),
  * an explicit (K x K) matrix form of the update (reference gdn2.py:10-11),
  * the third-party scalar gated delta rule of ``transformers`` (qwen3_next),
  * invariants the reference's own tests use (chunk-size and split/resume
    invariance, test_gdn2.py:111-152 and 185-233; causality),
  * central finite differences for the VJP,
and planted mistakes are shown to fail at least one pin.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import gdn2_oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"


def _rand(B, T, H, K, V, seed, decay="unit", h0=True):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, H, K))
    k = rng.standard_normal((B, T, H, K))
    v = rng.standard_normal((B, T, H, V))
    if decay == "unit":
        g = -np.abs(rng.random((B, T, H, K)))
    else:
        g = -np.logaddexp(0.0, rng.standard_normal((B, T, H, K)) + 2.0)
    b = 1 / (1 + np.exp(-rng.standard_normal((B, T, H, K))))
    w = 1 / (1 + np.exp(-rng.standard_normal((B, T, H, V))))
    s0 = rng.standard_normal((B, H, K, V)) * 0.1 if h0 else None
    return q, k, v, g, b, w, s0


def _matrix_form(q, k, v, g, b, w, s0):
    """S_t = (I - k (b*k)^T) Diag(e^g) S + k (w*v)^T ; o_t = S_t^T q  (explicit K x K matrices)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    qn = orc.l2normalize(q) * K**-0.5
    kn = orc.l2normalize(k)
    o = np.zeros((B, T, H, V))
    S = np.zeros((B, H, K, V)) if s0 is None else s0.copy()
    eye = np.eye(K)
    for bi in range(B):
        for h in range(H):
            St = S[bi, h]
            for t in range(T):
                kk = kn[bi, t, h][:, None]
                P = eye - kk @ (b[bi, t, h] * kn[bi, t, h])[None, :]
                St = P @ np.diag(np.exp(g[bi, t, h])) @ St + kk @ (w[bi, t, h] * v[bi, t, h])[None, :]
                o[bi, t, h] = St.T @ qn[bi, t, h]
            S[bi, h] = St
    return o, S


def test_linear_attention_closed_form():
    """b = 0, w = 1, g = 0: o = tril(q k^T) v with normalised, scaled q."""
    q, k, v, _, _, _, _ = _rand(2, 13, 3, 8, 5, seed=1, h0=False)
    z = np.zeros_like(q)
    o, S = orc.recurrent_fwd(q, k, v, z, z, np.ones_like(v))
    qn = orc.l2normalize(q) * 8**-0.5
    kn = orc.l2normalize(k)
    for bi in range(2):
        for h in range(3):
            A = np.tril(qn[bi, :, h] @ kn[bi, :, h].T)
            np.testing.assert_allclose(o[bi, :, h], A @ v[bi, :, h], rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(S[bi, h], kn[bi, :, h].T @ v[bi, :, h], atol=1e-12)


def test_single_token_closed_form():
    q, k, v, g, b, w, s0 = _rand(1, 1, 2, 6, 4, seed=2)
    o, S = orc.recurrent_fwd(q, k, v, g, b, w, s0)
    qn = orc.l2normalize(q)[0, 0] * 6**-0.5
    kn = orc.l2normalize(k)[0, 0]
    for h in range(2):
        Sd = np.exp(g[0, 0, h])[:, None] * s0[0, h]
        u = w[0, 0, h] * v[0, 0, h] - Sd.T @ (b[0, 0, h] * kn[h])
        exp_o = Sd.T @ qn[h] + (qn[h] @ kn[h]) * u
        np.testing.assert_allclose(o[0, 0, h], exp_o, atol=1e-13)
        np.testing.assert_allclose(S[0, h], Sd + np.outer(kn[h], u), atol=1e-13)
    # zero state: o = (q.k)(w*v)
    o0, _ = orc.recurrent_fwd(q, k, v, g, b, w, None)
    np.testing.assert_allclose(o0[0, 0], (qn * kn).sum(-1)[:, None] * (w * v)[0, 0], atol=1e-13)


def test_matches_explicit_matrix_form():
    args = _rand(2, 9, 2, 7, 5, seed=3, decay="paper")
    o1, s1 = orc.recurrent_fwd(*args)
    o2, s2 = _matrix_form(*args)
    np.testing.assert_allclose(o1, o2, atol=1e-12)
    np.testing.assert_allclose(s1, s2, atol=1e-12)


def test_matches_transformers_scalar_gated_delta_rule():
    """Broadcast scalar gates reduce gdn2 to the gated delta rule (third-party implementation)."""
    torch = pytest.importorskip("torch")
    qn3 = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    rng = np.random.default_rng(4)
    B, T, H, K, V = 2, 17, 3, 16, 12
    q = orc.l2normalize(rng.standard_normal((B, T, H, K)))
    k = orc.l2normalize(rng.standard_normal((B, T, H, K)))
    v = rng.standard_normal((B, T, H, V))
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
    gs = -np.logaddexp(0.0, rng.standard_normal((B, T, H)) + 2.0)
    s0 = rng.standard_normal((B, H, K, V)) * 0.1
    o, S = orc.recurrent_fwd(q, k, v, np.repeat(gs[..., None], K, -1), np.repeat(beta[..., None], K, -1),
                             np.repeat(beta[..., None], V, -1), s0, use_qk_l2norm_in_kernel=False)
    t = lambda x: torch.tensor(x, dtype=torch.float64)  # noqa: E731
    ot, St = qn3.torch_recurrent_gated_delta_rule(t(q), t(k), t(v), t(gs), t(beta), t(s0), True,
                                                  use_qk_l2norm_in_kernel=False)
    # that implementation casts to float32 internally
    assert orc.rel_l2(ot.numpy(), o) < 1e-6
    assert orc.rel_l2(St.numpy(), S) < 1e-6


@pytest.mark.parametrize("chunk", [1, 4, 8, 16, 33, 64])
@pytest.mark.parametrize("T", [8, 41, 100])
def test_chunk_form_equals_recurrence(chunk, T):
    args = _rand(2, T, 2, 16, 12, seed=T + chunk, decay="paper")
    o1, s1 = orc.recurrent_fwd(*args)
    o2, s2 = orc.chunk_fwd(*args, chunk_size=chunk)
    np.testing.assert_allclose(o2, o1, atol=1e-11)
    np.testing.assert_allclose(s2, s1, atol=1e-11)


def test_split_resume_and_causality():
    q, k, v, g, b, w, s0 = _rand(2, 12, 3, 16, 16, seed=5)
    o, s = orc.recurrent_fwd(q, k, v, g, b, w, s0)
    _, s_pre = orc.recurrent_fwd(q[:, :5], k[:, :5], v[:, :5], g[:, :5], b[:, :5], w[:, :5], s0)
    o_post, s_post = orc.chunk_fwd(q[:, 5:], k[:, 5:], v[:, 5:], g[:, 5:], b[:, 5:], w[:, 5:], s_pre,
                                   chunk_size=4)
    np.testing.assert_allclose(o[:, 5:], o_post, atol=1e-12)
    np.testing.assert_allclose(s, s_post, atol=1e-12)
    # appending tokens never changes earlier outputs
    o_short, _ = orc.recurrent_fwd(q[:, :7], k[:, :7], v[:, :7], g[:, :7], b[:, :7], w[:, :7], s0)
    np.testing.assert_allclose(o[:, :7], o_short, atol=1e-14)


def test_varlen_equals_separate_sequences():
    q, k, v, g, b, w, _ = _rand(1, 30, 2, 8, 8, seed=6)
    cu = [0, 4, 4, 19, 30]
    s0 = np.random.default_rng(7).standard_normal((4, 2, 8, 8)) * 0.1
    o, s = orc.recurrent_fwd(q, k, v, g, b, w, s0, cu_seqlens=cu)
    for n in range(4):
        a, e = cu[n], cu[n + 1]
        on, sn = orc.recurrent_fwd(q[:, a:e], k[:, a:e], v[:, a:e], g[:, a:e], b[:, a:e], w[:, a:e], s0[n:n + 1])
        np.testing.assert_allclose(o[:, a:e], on, atol=1e-14)
        np.testing.assert_allclose(s[n], sn[0], atol=1e-14)


def test_gva_equals_repeated_heads():
    rng = np.random.default_rng(8)
    B, T, H, HV, K, V = 1, 9, 2, 4, 8, 8
    q, k = rng.standard_normal((B, T, H, K)), rng.standard_normal((B, T, H, K))
    v, w = rng.standard_normal((B, T, HV, V)), rng.random((B, T, HV, V))
    g, b = -rng.random((B, T, HV, K)), rng.random((B, T, HV, K))
    o1, s1 = orc.recurrent_fwd(q, k, v, g, b, w)
    o2, s2 = orc.recurrent_fwd(np.repeat(q, 2, 2), np.repeat(k, 2, 2), v, g, b, w)
    np.testing.assert_allclose(o1, o2, atol=1e-14)
    np.testing.assert_allclose(s1, s2, atol=1e-14)


def test_pooled_identity_slots_reduce_to_recurrence():
    """Slots n -> n with one token per sequence: the pooled op is the plain op."""
    q, k, v, g, b, w, s0 = _rand(5, 1, 2, 8, 6, seed=21)
    o_ref, s_ref = orc.recurrent_fwd(q, k, v, g, b, w, s0)
    o, pool, written = orc.recurrent_fwd_pooled(q, k, v, g, b, w, s0, np.arange(5))
    np.testing.assert_allclose(o, o_ref, atol=1e-14)
    np.testing.assert_allclose(pool, s_ref, atol=1e-14)
    assert written == list(range(5))


def test_pooled_permuted_slots_and_padding():
    """Slots are a permutation into a larger pool; a padded entry (-1) starts from zero and
    stores nothing; untouched slots keep their contents."""
    q, k, v, g, b, w, _ = _rand(4, 3, 2, 8, 6, seed=22)
    rng = np.random.default_rng(23)
    pool = rng.standard_normal((9, 2, 8, 6))
    slots = np.array([[7, 7, 7], [2, 2, 2], [-1, -1, -1], [5, 5, 5]])
    o, new, written = orc.recurrent_fwd_pooled(q, k, v, g, b, w, pool, slots)
    assert written == [2, 5, 7]
    for n, sl in enumerate(slots[:, 0]):
        h0 = np.zeros((1, 2, 8, 6)) if sl < 0 else pool[sl][None]
        on, sn = orc.recurrent_fwd(q[n:n + 1], k[n:n + 1], v[n:n + 1], g[n:n + 1], b[n:n + 1],
                                   w[n:n + 1], h0)
        np.testing.assert_allclose(o[n], on[0], atol=1e-14)
        if sl >= 0:
            np.testing.assert_allclose(new[sl], sn[0], atol=1e-14)
    for r in (0, 1, 3, 4, 6, 8):
        np.testing.assert_array_equal(new[r], pool[r])


def test_speculative_resume_equals_accepted_prefix():
    """Speculative decoding: step 1 stores the state after each draft token t in slot
    idx[n, t]; step 2 resumes from slot idx[n, a_n - 1].  Its outputs must equal the plain
    recurrence over the a_n accepted tokens of step 1 followed by the step-2 tokens."""
    H, K, V, Tm = 2, 8, 6, 4
    rng = np.random.default_rng(24)
    s0 = rng.standard_normal((3, H, K, V)) * 0.3
    slots = np.array([[0, 1, 2, 3], [4, 5, 6, 7], [8, 9, 10, 11]])
    pool = np.zeros((12, H, K, V))
    pool[slots[:, 0]] = s0  # each sequence's current state sits in its first slot
    acc1 = np.array([1, 1, 1])
    step1 = _rand(1, 3 * Tm, H, K, V, seed=25)[:6]
    cu1 = [0, Tm, 2 * Tm, 3 * Tm]
    _, pool1, _ = orc.recurrent_fwd_pooled(*step1, pool, slots, acc1, cu_seqlens=cu1)
    acc2 = np.array([3, 1, 4])
    lens2 = [2, 3, 1]
    cu2 = np.concatenate([[0], np.cumsum(lens2)])
    step2 = _rand(1, int(cu2[-1]), H, K, V, seed=26)[:6]
    o2, pool2, _ = orc.recurrent_fwd_pooled(*step2, pool1, slots, acc2, cu_seqlens=cu2)
    for n in range(3):
        a = acc2[n]
        prefix = [x[:, cu1[n]:cu1[n] + a] for x in step1]
        new = [x[:, cu2[n]:cu2[n + 1]] for x in step2]
        joined = [np.concatenate([pa, pb], axis=1) for pa, pb in zip(prefix, new)]
        o_ref, s_ref, states = orc.recurrent_fwd(*joined, s0[n:n + 1], return_states=True)
        np.testing.assert_allclose(o2[:, cu2[n]:cu2[n + 1]], o_ref[:, a:], atol=1e-13)
        for t in range(lens2[n]):
            np.testing.assert_allclose(pool2[slots[n, t]], states[0][a + t], atol=1e-13)


def test_pooled_token_rows_and_transposed_layout():
    """Without in-place stores the state after token t goes to row bos + t, which equals the
    recurrence truncated after that token; the transposed layout is the swapped axes."""
    q, k, v, g, b, w, s0 = _rand(2, 3, 2, 8, 6, seed=27)
    _, _, states = orc.recurrent_fwd(q, k, v, g, b, w, s0, return_states=True)
    o, rows, written = orc.recurrent_fwd_pooled(q, k, v, g, b, w, s0, np.array([0, 1]),
                                                inplace_final_state=False, final_rows=6)
    assert written == list(range(6))
    for n in range(2):
        for t in range(3):
            np.testing.assert_allclose(rows[n * 3 + t], states[n][t], atol=1e-14)
    o_t, pool_t, _ = orc.recurrent_fwd_pooled(q, k, v, g, b, w, np.swapaxes(s0, -1, -2),
                                              np.array([1, 0]), transpose_state_layout=True)
    o_p, pool_p, _ = orc.recurrent_fwd_pooled(q, k, v, g, b, w, s0, np.array([1, 0]))
    np.testing.assert_allclose(o_t, o_p, atol=1e-14)
    np.testing.assert_allclose(pool_t, np.swapaxes(pool_p, -1, -2), atol=1e-14)


def test_short_conv_equals_numpy_convolution():
    """Per channel: the causal depthwise conv is numpy's full convolution with the kernel
    flipped (conv1d is a correlation), truncated to the first T outputs."""
    rng = np.random.default_rng(31)
    B, T, D, W = 2, 11, 5, 4
    x, w, bias = rng.standard_normal((B, T, D)), rng.standard_normal((D, W)), rng.standard_normal(D)
    y, new = orc.short_conv(x, w, bias, activation=None, output_final_state=True)
    for b in range(B):
        for d in range(D):
            ref = np.convolve(x[b, :, d], w[d, ::-1])[:T] + bias[d]
            np.testing.assert_allclose(y[b, :, d], ref, atol=1e-12)
    np.testing.assert_array_equal(new, np.transpose(x[:, -(W - 1):, :], (0, 2, 1)))
    ys, _ = orc.short_conv(x, w, bias)
    np.testing.assert_allclose(ys, y / (1 + np.exp(-y)), atol=1e-14)
    # Shorter than the kernel: the new cache keeps every input.
    _, new2 = orc.short_conv(x[:, :2], w, output_final_state=True)
    np.testing.assert_array_equal(new2, np.transpose(x[:, :2], (0, 2, 1)))


def test_short_conv_decode_step_continues_prefill():
    """A single-token call with the cache of the previous W-1 tokens equals the last row of
    the convolution over those tokens followed by the new one."""
    rng = np.random.default_rng(32)
    B, D, W = 3, 6, 4
    prev, tok = rng.standard_normal((B, W - 1, D)), rng.standard_normal((B, 1, D))
    w, bias = rng.standard_normal((D, W)), rng.standard_normal(D)
    _, cache = orc.short_conv(prev, w, bias, output_final_state=True)
    y1, new = orc.short_conv(tok, w, bias, cache=cache, output_final_state=True)
    yfull, _ = orc.short_conv(np.concatenate([prev, tok], 1), w, bias)
    np.testing.assert_allclose(y1[:, 0], yfull[:, -1], atol=1e-13)
    np.testing.assert_array_equal(new, np.transpose(np.concatenate([prev, tok], 1)[:, 1:], (0, 2, 1)))


def test_gated_rmsnorm_equals_torch_rms_norm():
    import torch

    rng = np.random.default_rng(33)
    x, z, w = rng.standard_normal((7, 64)) * 3, rng.standard_normal((7, 64)), rng.standard_normal(64)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (64,), torch.from_numpy(w), eps=1e-5)
    ref = ref * torch.nn.functional.silu(torch.from_numpy(z))
    np.testing.assert_allclose(orc.gated_rmsnorm(x, z, w, 1e-5), ref.numpy(), rtol=1e-12, atol=1e-12)


def test_rmsnorm_equals_torch_rms_norm():
    """The plain norm against torch's library rms_norm in float64, and its defining
    property: with unit weight and eps = 0 every row has unit root mean square."""
    import torch

    rng = np.random.default_rng(34)
    x, w = rng.standard_normal((9, 1024)) * 3, rng.standard_normal(1024)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (1024,), torch.from_numpy(w), eps=1e-5)
    np.testing.assert_allclose(orc.rmsnorm(x, w, 1e-5), ref.numpy(), rtol=1e-12, atol=1e-12)
    y = orc.rmsnorm(x, np.ones(1024), 0.0)
    np.testing.assert_allclose(np.sqrt((y * y).mean(-1)), 1.0, rtol=1e-12)


def test_vjp_matches_finite_differences():
    q, k, v, g, b, w, s0 = _rand(1, 11, 2, 6, 5, seed=9, decay="paper")
    rng = np.random.default_rng(10)
    do = rng.standard_normal(v.shape)
    dht = rng.standard_normal(s0.shape)
    grads = orc.recurrent_vjp(q, k, v, g, b, w, do, dht, s0)
    args = [q, k, v, g, b, w, s0]

    def loss(a):
        o, s = orc.recurrent_fwd(*a)
        return float((o * do).sum() + (s * dht).sum())

    for i, gr in enumerate(grads):
        d = rng.standard_normal(args[i].shape)
        eps = 1e-6
        ap = list(args)
        ap[i] = args[i] + eps * d
        am = list(args)
        am[i] = args[i] - eps * d
        fd = (loss(ap) - loss(am)) / (2 * eps)
        assert abs(fd - float((gr * d).sum())) <= 1e-6 * max(1.0, abs(fd)), i


def test_vjp_without_l2norm_matches_finite_differences():
    q, k, v, g, b, w, s0 = _rand(1, 7, 1, 5, 4, seed=11)
    rng = np.random.default_rng(12)
    do = rng.standard_normal(v.shape)
    grads = orc.recurrent_vjp(q, k, v, g, b, w, do, None, s0, use_qk_l2norm_in_kernel=False)
    for i, name in enumerate("qk"):
        d = rng.standard_normal(q.shape)
        a = [q, k]

        def L(x):
            aa = list(a)
            aa[i] = x
            o, _ = orc.recurrent_fwd(aa[0], aa[1], v, g, b, w, s0, use_qk_l2norm_in_kernel=False)
            return float((o * do).sum())

        eps = 1e-6
        fd = (L(a[i] + eps * d) - L(a[i] - eps * d)) / (2 * eps)
        assert abs(fd - float((grads[i] * d).sum())) <= 1e-6 * max(1.0, abs(fd)), name


@pytest.mark.parametrize("T,C", [(50, 16), (37, 8), (70, 64), (64, 64), (9, 4)])
def test_chunk_vjp_equals_recurrent_vjp(T, C):
    """The chunkwise backward algebra (reverse state scan, per-chunk products,
    reverse cumsum of dg) reproduces the token-serial derivative, ragged tails included."""
    q, k, v, g, b, w, s0 = _rand(2, T, 2, 8, 6, seed=20 + T, decay="paper")
    rng = np.random.default_rng(T)
    do = rng.standard_normal(v.shape)
    dht = rng.standard_normal(s0.shape)
    ref = orc.recurrent_vjp(q, k, v, g, b, w, do, dht, s0)
    got = orc.chunk_vjp(q, k, v, g, b, w, do, dht, s0, chunk_size=C)
    for name, a, r in zip(("dq", "dk", "dv", "dg", "db", "dw", "dh0"), got, ref):
        assert orc.rel_l2(a, r) < 1e-12, name


def test_chunk_vjp_without_l2norm_and_state():
    q, k, v, g, b, w, _ = _rand(1, 33, 1, 5, 4, seed=31, decay="unit")
    do = np.random.default_rng(32).standard_normal(v.shape)
    ref = orc.recurrent_vjp(q, k, v, g, b, w, do, None, None, use_qk_l2norm_in_kernel=False)
    got = orc.chunk_vjp(q, k, v, g, b, w, do, None, None, use_qk_l2norm_in_kernel=False, chunk_size=16)
    for a, r in zip(got, ref):
        assert orc.rel_l2(a, r) < 1e-12


def test_golden_fixtures_reproduce():
    f = np.load(GOLDEN / "gdn2_fwd_T100_H2_K32_V16.npz")
    x = {n: f[n].astype(np.float64) for n in ("q", "k", "v", "g", "b", "w", "h0")}
    o, ht = orc.recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["b"], x["w"], x["h0"])
    np.testing.assert_allclose(o, f["o"], atol=1e-12)
    np.testing.assert_allclose(ht, f["ht"], atol=1e-12)
    f = np.load(GOLDEN / "gdn2_varlen_T90_N4.npz")
    x = {n: f[n].astype(np.float64) for n in ("q", "k", "v", "g", "b", "w", "h0")}
    o, ht = orc.recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["b"], x["w"], x["h0"],
                              cu_seqlens=f["cu_seqlens"])
    np.testing.assert_allclose(o, f["o"], atol=1e-12)
    f = np.load(GOLDEN / "gdn2_bwd_T24_H2_K8_V8.npz")
    x = {n: f[n].astype(np.float64) for n in ("q", "k", "v", "g", "b", "w", "h0", "do", "dht")}
    grads = orc.recurrent_vjp(x["q"], x["k"], x["v"], x["g"], x["b"], x["w"], x["do"], x["dht"], x["h0"])
    for name, gr in zip(("dq", "dk", "dv", "dg", "db", "dw", "dh0"), grads):
        np.testing.assert_allclose(gr, f[name], atol=1e-12, err_msg=name)


def test_config0_recipe_and_fingerprint():
    inp = orc.make_inputs(0, 1, 512, 4, 64, 64)
    assert np.allclose(np.linalg.norm(inp["q"], axis=-1), 1.0)
    assert (inp["g"] < 0).all() and (inp["b"][..., :1] == inp["w"][..., :1]).all()
    f = np.load(GOLDEN / "gdn2_config0_fingerprint.npz")
    sums = np.array([float(np.sum(inp[n])) for n in ("q", "k", "v", "g", "b", "w")])
    np.testing.assert_allclose(sums, f["input_sums"], rtol=1e-12)
    o, ht = orc.recurrent_fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["b"], inp["w"])
    np.testing.assert_allclose(o[0, :64, 0], f["o_head0_first64"], atol=1e-12)
    np.testing.assert_allclose(ht, f["ht"], atol=1e-12)


def test_c_port_matches_oracle():
    from oracle import cpu_lib

    args = _rand(2, 37, 3, 24, 20, seed=13, decay="paper")
    o1, s1 = orc.recurrent_fwd(*args)
    o2, s2 = cpu_lib.recurrent_fwd_f32(*args[:6], h0=args[6], nthreads=2)
    assert orc.rel_l2(o2, o1) < 1e-5 and orc.rel_l2(s2, s1) < 1e-5


@pytest.mark.parametrize("fn", ["recurrent_fwd", "chunk_fwd"])
def test_torch_restatement_matches_oracle(fn):
    """The float32 PyTorch CPU restatement (the timed CPU baseline) equals the float64
    oracle, with a state, ragged chunk tails and the BASELINE decay distribution."""
    import torch

    from oracle import gdn2_torch

    args = _rand(2, 150, 3, 24, 20, seed=15, decay="paper")
    o1, s1 = orc.recurrent_fwd(*args)
    t = [torch.from_numpy(np.ascontiguousarray(a)).float() for a in args]
    o2, s2 = getattr(gdn2_torch, fn)(*t[:6], initial_state=t[6])
    assert o2.dtype == torch.float32 and s2.shape == (2, 3, 24, 20)
    assert orc.rel_l2(o2.double().numpy(), o1) < 1e-5 and orc.rel_l2(s2.double().numpy(), s1) < 1e-5


def test_torch_restatement_config0():
    """Both torch restatements on the config-0 workload against the committed fixture."""
    import torch

    from oracle import gdn2_torch

    inp = orc.make_inputs(0, 1, 512, 4, 64, 64)
    f = np.load(GOLDEN / "gdn2_config0_fingerprint.npz")
    t = [torch.from_numpy(inp[n]).float() for n in ("q", "k", "v", "g", "b", "w")]
    for fn in (gdn2_torch.recurrent_fwd, gdn2_torch.chunk_fwd):
        o, ht = fn(*t)
        assert orc.rel_l2(ht.double().numpy(), f["ht"]) < 1e-5
        assert orc.rel_l2(o[0, :64, 0].double().numpy(), f["o_head0_first64"]) < 1e-5


# ---------------------------------------------------------------- planted bugs
def _mutant(kind, q, k, v, g, b, w, s0):
    """The recurrence with one plausible mistake (used only to show the pins bite)."""
    B, T, H, K = q.shape
    qn = orc.l2normalize(q) * K**-0.5
    kn = orc.l2normalize(k)
    o = np.zeros((B, T, H, v.shape[-1]))
    S = np.zeros((B, H, K, v.shape[-1])) if s0 is None else s0.copy()
    for t in range(T):
        a = np.exp(g[:, t])[..., None]
        e = b[:, t] * kn[:, t]
        if kind == "erase_before_decay":
            r = np.einsum("bhkv,bhk->bhv", S, e)
            S = S * a
        else:
            S = S * a
            r = np.einsum("bhkv,bhk->bhv", S, kn[:, t] if kind == "erase_without_b" else e)
        u = w[:, t] * v[:, t] - r
        S_new = S + kn[:, t][..., None] * u[..., None, :]
        o[:, t] = np.einsum("bhkv,bhk->bhv", S if kind == "read_before_write" else S_new, qn[:, t])
        S = S_new
    return o, S


@pytest.mark.parametrize("kind", ["erase_before_decay", "erase_without_b", "read_before_write"])
def test_planted_mistakes_fail_the_matrix_form_pin(kind):
    args = _rand(1, 6, 2, 6, 4, seed=14, decay="paper")
    o_ref, _ = _matrix_form(*args)
    o_bad, _ = _mutant(kind, *args)
    o_good, _ = _mutant("none", *args)
    np.testing.assert_allclose(o_good, o_ref, atol=1e-12)
    assert np.abs(o_bad - o_ref).max() > 1e-6
