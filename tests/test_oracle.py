"""Pins the CPU oracle (oracle/) before anything is checked against it.

The reference ships no golden vectors (its only check is a runtime comparison
with BaselineTransformer, torch_transformer_benchmark.py:1307-1372), so the
restated baseline is pinned by an independent float64 brute force, by
invariants the causal pre-norm block must satisfy, and by planted mistakes
that those checks have to catch.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import numpy_ref
from oracle.accuracy import compare_outputs
from oracle.baseline import BaselineSelfAttention, BaselineTransformer, generate_random_case


class Cfg:
    def __init__(self, b, s, d, h, f, layers, causal=True):
        self.batch_size, self.seq_len, self.d_model = b, s, d
        self.num_heads, self.ffn_dim, self.num_layers, self.causal = h, f, layers, causal


def _model(cfg, seed=1234, randomize_norms=True):
    torch.manual_seed(seed)
    model = BaselineTransformer(cfg).eval()
    if randomize_norms:  # exercise the affine path too
        with torch.no_grad():
            for name, p in model.named_parameters():
                if "norm" in name:
                    p.copy_(torch.randn_like(p) * 0.2 + (1.0 if name.endswith("weight") else 0.0))
    return model


def _torch_f64(model, x):
    m64 = BaselineTransformer(model.config)
    m64.load_state_dict(model.state_dict())
    m64 = m64.double().eval()
    with torch.no_grad():
        return m64(x.double()).numpy()


@pytest.mark.parametrize("geom", [(2, 5, 16, 2, 24, 2), (1, 9, 32, 4, 32, 1), (2, 7, 32, 1, 16, 2), (1, 6, 16, 2, 8, 3)])
def test_baseline_matches_float64_brute_force(geom):
    cfg = Cfg(*geom)
    model = _model(cfg)
    x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=torch.Generator().manual_seed(7))
    expected = numpy_ref.forward(numpy_ref.state_to_numpy(model.state_dict()), x.numpy(), cfg.num_layers, cfg.num_heads)
    got64 = _torch_f64(model, x)
    # Even in float64 the baseline runs its softmax on scores.float() (TTB:256),
    # so the float64 restatement agrees with the brute force to ~1e-7, not 1e-12.
    np.testing.assert_allclose(got64, expected, rtol=1e-6, atol=1e-6)
    with torch.no_grad():
        got32 = model(x).numpy()
    np.testing.assert_allclose(got32, expected, rtol=1e-4, atol=1e-4)


def test_non_causal_brute_force():
    cfg = Cfg(1, 6, 16, 2, 16, 1, causal=False)
    model = _model(cfg)
    x = torch.randn(1, 6, 16, generator=torch.Generator().manual_seed(3))
    expected = numpy_ref.forward(numpy_ref.state_to_numpy(model.state_dict()), x.numpy(), 1, 2, causal=False)
    np.testing.assert_allclose(_torch_f64(model, x), expected, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("mistake", ["diagonal", "tanh_gelu", "no_scale", "ln_gain"])
def test_brute_force_rejects_planted_mistakes(mistake, monkeypatch):
    """Each plausible slip in the restatement must be visible to the brute force."""
    cfg = Cfg(2, 6, 16, 2, 16, 2)
    model = _model(cfg)
    x = torch.randn(2, 6, 16, generator=torch.Generator().manual_seed(11))
    state = numpy_ref.state_to_numpy(model.state_dict())
    good = numpy_ref.forward(state, x.numpy(), 2, 2)

    if mistake == "diagonal":  # strict mask: a token may not attend to itself
        def attn(q, k, v, h, causal=True):
            out = np.zeros_like(q)
            hd = q.shape[-1] // h
            for b in range(q.shape[0]):
                for hh in range(h):
                    c = slice(hh * hd, (hh + 1) * hd)
                    for i in range(q.shape[1]):
                        last = max(i, 1)
                        s = np.array([q[b, i, c] @ k[b, j, c] * hd**-0.5 for j in range(last)])
                        w = np.exp(s - s.max()); w /= w.sum()
                        out[b, i, c] = w @ v[b, :last, c]
            return out
        monkeypatch.setattr(numpy_ref, "causal_attention", attn)
    elif mistake == "tanh_gelu":
        monkeypatch.setattr(numpy_ref, "gelu_erf", lambda z: 0.5 * z * (1 + np.tanh(math.sqrt(2 / math.pi) * (z + 0.044715 * z**3))))
    elif mistake == "no_scale":
        original = numpy_ref.causal_attention
        monkeypatch.setattr(numpy_ref, "causal_attention", lambda q, k, v, h, causal=True: original(q * math.sqrt(q.shape[-1] // h), k, v, h, causal))
    elif mistake == "ln_gain":
        original_ln = numpy_ref.layer_norm
        monkeypatch.setattr(numpy_ref, "layer_norm", lambda z, g, b, eps=1e-5: original_ln(z, g, b, eps) * 1.01)
    bad = numpy_ref.forward(state, x.numpy(), 2, 2)
    # The check that pins the FP32 restatement (1e-4 above) must reject it.
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(bad, good, rtol=1e-4, atol=1e-4)


def _compacted_reference(model, x, mask):
    """Run each sequence's valid tokens alone, in order, and scatter them back.

    Without positional encodings a padded token enters the baseline only as a
    masked key, so a padded forward must equal the forward over the valid
    tokens compacted into a shorter sequence (causal order is kept), with the
    padded rows zero.
    """
    out = torch.zeros_like(x)
    for b in range(x.shape[0]):
        idx = torch.nonzero(mask[b]).flatten()
        if idx.numel() == 0:
            continue
        model.config = Cfg(1, idx.numel(), x.shape[2], model.config.num_heads, model.config.ffn_dim,
                           model.config.num_layers, model.config.causal)
        with torch.no_grad():
            out[b, idx] = model(x[b : b + 1, idx].contiguous())[0]
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_padding_equals_compaction(causal):
    """Pins the restated padding semantics (TTB:250-253, :263-264, :290-291, :314-315)."""
    cfg = Cfg(4, 12, 32, 4, 48, 2, causal)
    model = _model(cfg)
    x = torch.randn(4, 12, 32, generator=torch.Generator().manual_seed(17))
    mask = torch.ones(4, 12, dtype=torch.bool)
    mask[0, 9:] = False            # right padding
    mask[1, :5] = False            # left padding (causal: padded queries see no key)
    mask[2, ::2] = False           # holes
    mask[3, :] = False             # nothing valid
    with torch.no_grad():
        padded = model(x, mask)
    assert torch.isfinite(padded).all()
    expected = _compacted_reference(model, x, mask)
    model.config = cfg
    torch.testing.assert_close(padded, expected, atol=1e-5, rtol=1e-5)

    # Planted mistake: zeroing padded outputs without masking them as keys.
    original = BaselineSelfAttention.forward

    def keys_unmasked(self, xx, valid_token_mask=None, causal=False):
        out = original(self, xx, None, causal)
        return out if valid_token_mask is None else out.masked_fill(~valid_token_mask[..., None], 0)

    BaselineSelfAttention.forward = keys_unmasked
    try:
        with torch.no_grad():
            bad = model(x, mask)
    finally:
        BaselineSelfAttention.forward = original
    assert not torch.allclose(bad, expected, atol=1e-3, rtol=1e-3)


def test_causal_prefix_invariance():
    """out[:, :p] depends only on x[:, :p] (the basis of cfg5's prefix check)."""
    cfg = Cfg(2, 24, 32, 4, 32, 2)
    model = _model(cfg)
    x = torch.randn(2, 24, 32, generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        full = model(x)
        p = 10
        short_cfg = Cfg(2, p, 32, 4, 32, 2)
        model.config = short_cfg
        prefix = model(x[:, :p].contiguous())
        model.config = cfg
    torch.testing.assert_close(full[:, :p], prefix, rtol=1e-5, atol=1e-5)


def test_batch_independence():
    cfg = Cfg(3, 12, 32, 2, 32, 2)
    model = _model(cfg)
    x = torch.randn(3, 12, 32, generator=torch.Generator().manual_seed(9))
    with torch.no_grad():
        full = model(x)
        single = model(x[1:2].contiguous())
    torch.testing.assert_close(full[1:2], single, rtol=1e-5, atol=1e-5)


def test_single_token_attention_closed_form():
    """With S=1 softmax is 1, so attention reduces to out_proj(v_proj(x))."""
    torch.manual_seed(0)
    att = BaselineSelfAttention(16, 4).eval()
    x = torch.randn(3, 1, 16)
    with torch.no_grad():
        got = att(x, None, causal=True)
        want = att.out_proj(att.v_proj(x))
    torch.testing.assert_close(got, want, rtol=1e-6, atol=1e-6)


def test_layer_norm_row_statistics():
    torch.manual_seed(0)
    cfg = Cfg(1, 4, 64, 4, 64, 1)
    model = BaselineTransformer(cfg).eval()
    x = torch.randn(1, 4, 64) * 3 + 1
    with torch.no_grad():
        y = model.final_norm(x)
    torch.testing.assert_close(y.mean(-1), torch.zeros(1, 4), atol=1e-5, rtol=0)
    torch.testing.assert_close(y.var(-1, unbiased=False), torch.ones(1, 4), atol=1e-3, rtol=0)


def test_numpy_ref_textbook_identities():
    z = np.linspace(-4, 4, 17)
    gelu = numpy_ref.gelu_erf(z)
    np.testing.assert_allclose(gelu, [0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in z], rtol=1e-15)
    np.testing.assert_allclose(gelu, F.gelu(torch.from_numpy(z), approximate="none").numpy(), rtol=1e-12, atol=1e-14)
    x = np.random.default_rng(0).normal(size=(3, 8))
    ln = numpy_ref.layer_norm(x, np.ones(8), np.zeros(8), 0.0)
    np.testing.assert_allclose(ln.mean(-1), 0, atol=1e-12)
    np.testing.assert_allclose((ln**2).mean(-1), 1, atol=1e-12)
    # identical keys -> uniform weights -> context is the mean of the visible values
    q = np.random.default_rng(1).normal(size=(1, 5, 4))
    k = np.ones((1, 5, 4))
    v = np.arange(20, dtype=np.float64).reshape(1, 5, 4)
    ctx = numpy_ref.causal_attention(q, k, v, 1)
    for i in range(5):
        np.testing.assert_allclose(ctx[0, i], v[0, : i + 1].mean(0), rtol=1e-12)


# ----------------------------------------------------------------------------- accuracy rule
def test_compare_outputs_rule_edges():
    ref = torch.tensor([1.0, 0.0, 0.0, 10.0, 0.5, 0.0])
    opt = torch.tensor([1.002, 0.002, 0.0021, 10.19, 0.5 + 0.0115, float("nan")])
    r = compare_outputs(ref, opt, rtol=0.02, atol=0.002)
    # |d| == atol passes (<=); 0.0021 > atol at ref=0 fails; 0.19 <= 0.2 passes (rel);
    # 0.0115 > max(0.002, 0.01) fails although atol + rtol*|ref| = 0.012 (isclose would pass); NaN fails.
    assert r.failed_elements == 3
    assert r.failed_feature_dims == [2, 4, 5]
    assert not r.passed


def test_compare_outputs_reports_worst_index_and_inf():
    ref = torch.zeros(2, 3, 4)
    opt = ref.clone()
    opt[1, 2, 3] = 0.5
    r = compare_outputs(ref, opt)
    assert r.worst_index == (1, 2, 3) and r.failed_elements == 1 and r.failed_feature_dims == [3]
    opt2 = ref.clone()
    opt2[0, 0, 0] = float("inf")
    assert compare_outputs(ref, opt2).failed_elements == 1
    assert compare_outputs(ref, ref).passed


def test_compare_outputs_shape_mismatch():
    with pytest.raises(AssertionError):
        compare_outputs(torch.zeros(2, 3), torch.zeros(3, 2))


# ----------------------------------------------------------------------------- inputs
def test_generate_random_case_contract():
    cfg = Cfg(4, 32, 16, 2, 16, 1)
    x1, m1 = generate_random_case(cfg, torch.device("cpu"), torch.float32, seed=5)
    x2, _ = generate_random_case(cfg, torch.device("cpu"), torch.float32, seed=5)
    assert x1.shape == (4, 32, 16) and m1.dtype == torch.bool and bool(m1.all())
    assert torch.equal(x1, x2)
    direct = torch.randn(4, 32, 16, generator=torch.Generator().manual_seed(5))
    assert torch.equal(x1, direct)
    xp, mp = generate_random_case(cfg, torch.device("cpu"), torch.float32, seed=5, padding_ratio=0.25)
    lengths = mp.sum(1)
    assert int(lengths.min()) >= round(32 * 0.75) and int(lengths.max()) <= 32
    assert bool((xp[~mp] == 0).all())
    assert bool(mp[:, 0].all())


# ----------------------------------------------------------------------------- GELU approximation
GELU_C = (1.59501577, 0.0740112920, -7.03033577e-4)


def _gelu_device(x: np.ndarray) -> np.ndarray:
    """float64 restatement of the device GELU (common.h): x * logistic(c1 x + c3 x^3 + c5 x^5), x clamped to +-9."""
    xc = np.clip(x, -9.0, 9.0)
    z = xc * (GELU_C[0] + xc * xc * (GELU_C[1] + xc * xc * GELU_C[2]))
    return x / (1.0 + np.exp(-z))


def test_gelu_approximation_error_bound():
    """|device GELU - exact erf GELU| <= 3e-5 everywhere, far below one FP16 ulp of the stored activation."""
    for lo, hi, n in ((-12.0, 12.0, 400001), (-200.0, 200.0, 400001)):
        x = np.linspace(lo, hi, n)
        exact = numpy_ref.gelu_erf(x)
        err = np.abs(_gelu_device(x) - exact)
        assert err.max() < 3e-5, (lo, hi, err.max())
    huge = np.array([-1e6, -1e3, -9.5, 9.5, 1e3, 1e6])
    np.testing.assert_allclose(_gelu_device(huge), numpy_ref.gelu_erf(huge), rtol=1e-9, atol=1e-5)
    # the quintic term matters: the plain x, x^3 logistic (the tanh form the
    # reference's Triton epilogue used) is 15x further from exact erf
    x = np.linspace(-12.0, 12.0, 200001)
    exact = numpy_ref.gelu_erf(x)
    tanh_form = 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x**3)))
    assert np.abs(tanh_form - exact).max() > 1e-4
