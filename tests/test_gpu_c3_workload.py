"""Config 3's own workload (bf16, batch 4, a 2048-token prompt, then 256 greedy steps).

* **One gdn2 layer at config 3's module shape** (hidden 1024, 16 heads x 64, bf16, B = 4):
  the module's inference prefill over 2048 tokens, which takes the convolutions inside the
  chunk kernels (``ops.chunk_gdn2_conv``), then 256 single-token steps on the fused decode
  kernel (``ops.decode_step_fused``) with the caches updated in place.  Checked against
  the float64 oracle composition of the reference forward (``gdn2.py:815-999``) on the
  same bf16 weights and inputs: projections -> ``short_conv`` (with its cache on the
  steps) -> gate -> ``recurrent_fwd`` -> ``gated_rmsnorm`` -> ``o_proj``.  The bar is the
  bf16 one (rel. L2 <= 2e-2) on every output position, on the final recurrent state and
  on the three conv caches.
* **The full config-3 GreedyDecoder** (24 layers, 0.68 B parameters, bf16): B4 x 2048
  prompt + 256 greedy steps.  The graph-replayed decode gives the eager decode's tokens,
  and every step's logits are finite.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as orc
from tests._helpers import rel_l2

pytestmark = pytest.mark.gpu

B, T_PRE, N_STEPS, D, H, HD = 4, 2048, 256, 1024, 16, 64


def _oracle_layer(m, x):
    """Float64 composition of the module forward on CPU, streaming: a prefill over
    ``T_PRE`` tokens from zero history, then the remaining tokens one at a time with
    the conv caches (``short_conv`` with a cache on a single-token call) and the state.
    Returns outputs ``[B, T, D]``, the final state and the final conv caches."""
    P = {n: p.detach().double().cpu() for n, p in m.named_parameters()}
    xd = x.double().cpu()

    def lin(t, name):
        y = t @ P[name + ".weight"].T
        bias = P.get(name + ".bias")
        return y if bias is None else y + bias

    raw = [lin(xd, n).numpy() for n in ("q_proj", "k_proj", "v_proj")]
    taps = [P[f"{c}.conv1d.weight"].numpy() for c in ("q_conv1d", "k_conv1d", "v_conv1d")]
    A = np.repeat(np.exp(P["A_log"].numpy()), HD)
    f = lin(lin(xd, "f_proj.0"), "f_proj.1").numpy()
    g = -A * np.logaddexp(0.0, f + P["dt_bias"].numpy())
    b = 1.0 / (1.0 + np.exp(-lin(xd, "b_proj").numpy()))
    w = 1.0 / (1.0 + np.exp(-lin(xd, "w_proj").numpy()))
    z = lin(lin(xd, "g_proj.0"), "g_proj.1").numpy()
    heads = lambda t: t.reshape(*t.shape[:-1], H, HD)  # noqa: E731

    T = x.shape[1]
    conv = [orc.short_conv(r[:, :T_PRE], wt, None, None, True, "silu") for r, wt in zip(raw, taps)]
    qkv = [[c[0]] for c in conv]
    caches = [c[1] for c in conv]
    for t in range(T_PRE, T):
        for i in range(3):
            y, caches[i] = orc.short_conv(raw[i][:, t:t + 1], taps[i], None, caches[i], True, "silu")
            qkv[i].append(y)
    q, k, v = (np.concatenate(parts, axis=1) for parts in qkv)
    o, state = orc.recurrent_fwd(heads(q), heads(k), heads(v), heads(g), heads(b), heads(w))
    o = orc.gated_rmsnorm(o, heads(z), P["o_norm.weight"].numpy(), m.o_norm.eps)
    out = o.reshape(B, T, -1) @ P["o_proj.weight"].numpy().T
    return out, state, caches


def test_c3_gdn2_layer_prefill_then_decode(gpu_device, monkeypatch):
    from qwendopamine_amd import GatedDeltaNet2, ops

    print("[case] config-3 gdn2 layer: bf16 B4 prefill 2048 + 256 fused decode steps", flush=True)
    calls = {"chunk_gdn2_conv": 0, "decode_step_fused": 0}
    for name in calls:
        fn = getattr(ops, name)

        def counted(*a, _fn=fn, _name=name, **kw):
            calls[_name] += 1
            return _fn(*a, **kw)

        monkeypatch.setattr(ops, name, counted)

    torch.manual_seed(3)
    m = GatedDeltaNet2(hidden_size=D, num_heads=H, head_dim=HD, layer_idx=0)
    m = m.to(gpu_device, torch.bfloat16).eval()
    gen = torch.Generator(device="cpu").manual_seed(3)
    x = torch.randn(B, T_PRE + N_STEPS, D, generator=gen).to(torch.bfloat16).to(gpu_device)
    cache: dict = {}
    with torch.no_grad():
        outs = [m(x[:, :T_PRE], past_key_values=cache, use_cache=True)[0]]
        state0 = cache["recurrent_state"]
        conv0 = cache["conv_state"]
        for t in range(T_PRE, T_PRE + N_STEPS):
            o, _, cache = m(x[:, t:t + 1], past_key_values=cache, use_cache=True, update_cache_in_place=True)
            outs.append(o)
    torch.cuda.synchronize()
    assert calls == {"chunk_gdn2_conv": 1, "decode_step_fused": N_STEPS}, calls
    # In place: the steps wrote into the prefill's cache tensors.
    assert cache["recurrent_state"].data_ptr() == state0.data_ptr()
    assert all(a.data_ptr() == c.data_ptr() for a, c in zip(cache["conv_state"], conv0))
    out = torch.cat(outs, 1).float().cpu().numpy()
    assert np.isfinite(out).all()

    ref_out, ref_state, ref_caches = _oracle_layer(m, x)
    per_pos = [orc.rel_l2(out[:, t], ref_out[:, t]) for t in range(out.shape[1])]
    worst = int(np.argmax(per_pos))
    e_state = rel_l2(cache["recurrent_state"], ref_state)
    e_conv = [rel_l2(c, r) for c, r in zip(cache["conv_state"], ref_caches)]
    print(f"  rel_l2 outputs: prefill max {max(per_pos[:T_PRE]):.2e}, decode max {max(per_pos[T_PRE:]):.2e} "
          f"(worst position {worst}); state {e_state:.2e}; conv caches "
          + ", ".join(f"{e:.2e}" for e in e_conv), flush=True)
    assert max(per_pos) <= 2e-2, (worst, per_pos[worst])
    assert e_state <= 2e-2
    assert max(e_conv) <= 2e-2


def test_c3_greedy_decoder_graph_equals_eager(gpu_device):
    from qwendopamine_amd.hybrid import GreedyDecoder, HybridConfig, HybridDecoder

    print("[case] config-3 GreedyDecoder bf16 B4 x 2048 + 256 steps, graph vs eager", flush=True)
    torch.manual_seed(3)
    cfg = HybridConfig.c3()
    m = HybridDecoder(cfg).to(gpu_device, torch.bfloat16).eval()
    gen = torch.Generator(device=gpu_device).manual_seed(3)
    prompt = torch.randint(0, cfg.vocab_size, (B, T_PRE), generator=gen, device=gpu_device)
    runs = {}
    for use_graph in (False, True):
        dec = GreedyDecoder(m, use_graph=use_graph, keep_logits=True)
        toks = [dec.prefill(prompt, N_STEPS).clone()]
        finite = [torch.isfinite(dec.logits).all()]
        maxabs = [dec.logits.abs().max()]
        last = dec.logits.clone()
        for _ in range(N_STEPS - 1):
            toks.append(dec.step().clone())
            finite.append(torch.isfinite(dec.logits).all())
            maxabs.append(dec.logits.abs().max())
        torch.cuda.synchronize()
        runs[use_graph] = (torch.cat(toks, 1), torch.stack(finite), torch.stack(maxabs), dec.logits.clone(), last)
        print(f"  use_graph={use_graph}: tokens {tuple(runs[use_graph][0].shape)}, "
              f"max |logit| {float(runs[use_graph][2].max()):.3g}", flush=True)
    (te, fe, _, le, pe), (tg, fg, _, lg, pg) = runs[False], runs[True]
    assert te.shape == (B, N_STEPS) and bool(fe.all()) and bool(fg.all())
    assert int(te.min()) >= 0 and int(te.max()) < cfg.vocab_size
    assert torch.equal(pe, pg)  # the prefill is the same eager call in both runs
    n_same = int((te == tg).all(0).long().cumprod(0).sum())
    print(f"  graph = eager for the first {n_same} of {N_STEPS} steps", flush=True)
    assert torch.equal(te, tg)
    assert rel_l2(lg, le) <= 1e-3
