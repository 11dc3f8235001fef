"""Pins the attention oracle (oracle.attention, the reference's chunked_forward
rows in float64) against torch's CPU math attention in float64, and against
closed forms: equal scores average v, a dominant key selects its value row,
fully masked rows give 0 / +inf, grouped-query heads read their kv head."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import oracle as orc


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def torch_ref(q, k, v, bias=None, causal=False, scale=None):
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    g = q.shape[1] // k.shape[1]
    kk, vv = t(k).repeat_interleave(g, 1), t(v).repeat_interleave(g, 1)
    mask = None if bias is None else t(np.broadcast_to(bias, q.shape[:3] + (k.shape[2],)))
    return F.scaled_dot_product_attention(t(q), kk, vv, attn_mask=mask, is_causal=causal, scale=scale).numpy()


def test_matches_torch_math_float64():
    q, k, v = rnd((2, 8, 37, 16), 0), rnd((2, 2, 53, 16), 1), rnd((2, 2, 53, 24), 2)
    bias = rnd((1, 8, 37, 53), 3)
    for causal, b in ((False, None), (True, None), (False, bias)):
        out, lse = orc.attention(q, k, v, b, causal)
        np.testing.assert_allclose(out, torch_ref(q, k, v, b, causal), rtol=1e-12, atol=1e-12)
    # lse against a direct logsumexp of the scores
    out, lse = orc.attention(q, k, v, None, False, scale=0.3)
    s = np.einsum("bhld,bhsd->bhls", q, np.repeat(k, 4, axis=1)) * 0.3
    np.testing.assert_allclose(lse, np.log(np.exp(s).sum(-1)), rtol=1e-12)


def test_closed_forms():
    v = rnd((1, 1, 10, 4), 4)
    q = np.zeros((1, 1, 3, 8))
    k = rnd((1, 1, 10, 8), 5)
    out, lse = orc.attention(q, k, v)                           # all scores 0: the mean of v
    np.testing.assert_allclose(out[0, 0], np.repeat(v[0, 0].mean(0, keepdims=True), 3, 0), rtol=1e-12)
    np.testing.assert_allclose(lse, np.log(10.0))
    bias = np.full((1, 1, 3, 10), -np.inf)
    bias[0, 0, 1, 7] = 0.0                                    # row 1 sees only key 7; rows 0, 2 see nothing
    out, lse = orc.attention(q, k, v, bias)
    np.testing.assert_allclose(out[0, 0, 1], v[0, 0, 7], rtol=1e-12)
    assert (out[0, 0, [0, 2]] == 0).all() and np.isinf(lse[0, 0, [0, 2]]).all() and lse[0, 0, 1] == 0.0
    out, _ = orc.attention(np.ones((1, 1, 4, 8)), np.ones((1, 1, 4, 8)), v[:, :, :4], causal=True)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0, 0], rtol=1e-12)   # causal row 0 sees key 0 only
    np.testing.assert_allclose(out[0, 0, 3], v[0, 0, :4].mean(0), rtol=1e-12)


def test_grouped_heads_read_their_kv_head():
    q, k, v = rnd((1, 4, 5, 8), 6), rnd((1, 2, 7, 8), 7), rnd((1, 2, 7, 8), 8)
    out, _ = orc.attention(q, k, v)
    for h in range(4):
        o1, _ = orc.attention(q[:, h:h + 1], k[:, h // 2:h // 2 + 1], v[:, h // 2:h // 2 + 1])
        np.testing.assert_allclose(out[:, h:h + 1], o1, rtol=1e-12)


def test_backward_matches_torch_autograd_float64():
    q, k, v = rnd((2, 4, 19, 8), 10), rnd((2, 2, 23, 8), 11), rnd((2, 2, 23, 8), 12)
    dout = rnd((2, 4, 19, 8), 13)
    bias = rnd((1, 4, 19, 23), 14)
    for causal, b in ((False, None), (True, None), (False, bias)):
        dq, dk, dv = orc.attention_bwd(q, k, v, dout, b, causal)
        tq, tk, tv = (torch.from_numpy(x).requires_grad_() for x in (q, k, v))
        mask = None if b is None else torch.from_numpy(np.broadcast_to(b, (2, 4, 19, 23)).copy())
        o = F.scaled_dot_product_attention(tq, tk.repeat_interleave(2, 1), tv.repeat_interleave(2, 1), attn_mask=mask,
                                           is_causal=causal)
        o.backward(torch.from_numpy(dout))
        for got, want in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
            np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-12)


def test_score_gradient_is_the_bias_gradient():
    # the oracle's dS, summed over a broadcast bias's dimensions, is torch autograd's bias gradient
    q, k, v = rnd((2, 4, 11, 8), 30), rnd((2, 2, 13, 8), 31), rnd((2, 2, 13, 8), 32)
    dout = rnd((2, 4, 11, 8), 33)
    for shape, causal in (((1, 4, 11, 13), False), ((2, 1, 11, 13), True), ((11, 13), False)):
        b = rnd(shape, 34)
        *_, ds = orc.attention_bwd(q, k, v, dout, b, causal, return_ds=True)
        assert ds.shape == (2, 4, 11, 13)
        tb = torch.from_numpy(b.copy()).requires_grad_()
        tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
        mask = tb
        if causal:
            # SDPA takes no mask together with is_causal: fold the causal mask into the bias
            mask = tb + torch.full((11, 13), float("-inf"), dtype=torch.float64).triu(1)
        o = F.scaled_dot_product_attention(tq, tk.repeat_interleave(2, 1), tv.repeat_interleave(2, 1), attn_mask=mask)
        o.backward(torch.from_numpy(dout))
        if len(shape) == 2:
            got = ds.sum(axis=(0, 1))
        else:
            got = ds.sum(axis=tuple(i for i, n in enumerate(shape) if n == 1), keepdims=True)
        np.testing.assert_allclose(got, tb.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_backward_rounding_option_changes_only_the_staged_values():
    # round_to rounds P and dS to the dtype: on inputs where both are exact in float16
    # (P in {0, 1} through a dominant key, dS small dyadic values) the rounded and exact results agree
    q = np.zeros((1, 1, 2, 8))
    k = np.zeros((1, 1, 2, 8))
    v = rnd((1, 1, 2, 8), 20)
    dout = np.full((1, 1, 2, 8), 0.5)
    bias = np.array([[[[0.0, -np.inf], [0.0, -np.inf]]]])
    exact = orc.attention_bwd(q, k, v, dout, bias)
    rounded = orc.attention_bwd(q, k, v, dout, bias, round_to=orc.F16)
    for a, b in zip(exact, rounded):
        np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)
    # and on random inputs it differs by about the dtype's rounding
    q, k, v, dout = rnd((1, 2, 16, 8), 21), rnd((1, 2, 16, 8), 22), rnd((1, 2, 16, 8), 23), rnd((1, 2, 16, 8), 24)
    e = orc.attention_bwd(q, k, v, dout)
    r = orc.attention_bwd(q, k, v, dout, round_to=orc.BF16)
    d = max(np.abs(a - b).max() for a, b in zip(e, r))
    assert 0 < d < 0.05
