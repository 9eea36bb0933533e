"""Pins the oracle's activation producers (zero/kernels/ops.cl:82-128, 2025-2075): closed forms, float64 references
of the norms and activations, and consistency with the pinned quantizer."""
import numpy as np

import oracle


def f64_rms(x, eps):
    x = x.astype(np.float64)
    return 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)


def test_rmsnorm_closed_forms_and_padding():
    K, eps = 512, 1e-6
    x = np.zeros((3, K), dtype=np.float32)
    x[0] = 2.5                      # constant row: y = c / sqrt(c^2 + eps)
    x[2, ::2] = 3.0                 # half the row: mean square 4.5
    w = np.ones(K, dtype=np.float32)
    aq, asc, absum, h = oracle.rmsnorm_quant(x, w, eps, M_stride=5)
    assert np.allclose(h[0], 2.5 / np.sqrt(6.25 + eps), rtol=2e-7)
    assert np.all(h[1] == 0) and np.all(aq[1] == 0) and np.all(asc[:, 1] == 0)   # zero row
    assert np.allclose(h[2, ::2], 3.0 / np.sqrt(4.5 + eps), rtol=2e-7) and np.all(h[2, 1::2] == 0)
    assert np.all(aq[3:] == 0) and np.all(h[3:] == 0) and np.all(asc[:, 3:] == 0)  # padding rows
    assert np.all(aq[0] == 127)     # a constant positive row quantizes to 127 everywhere


def test_rmsnorm_vs_float64_and_quantizer_consistency():
    rng = np.random.default_rng(1)
    K, eps = 2048, 1e-5
    x = (rng.standard_normal((4, K)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    aq, asc, absum, h = oracle.rmsnorm_quant(x, w, eps)
    ref = x.astype(np.float64) * f64_rms(x, eps) * w
    assert np.max(np.abs(h - ref) / np.max(np.abs(ref))) < 1e-6
    q2, s2, a2 = oracle.quantize_act(h)
    assert np.array_equal(q2, aq) and np.array_equal(s2, asc) and np.array_equal(a2, absum)


def test_swiglu_closed_forms_and_identities():
    F = 256
    g = np.zeros((4, 2 * F), dtype=np.float32)
    g[0, :F] = 0.0
    g[0, F:] = 5.0                    # silu(0) = 0
    g[1, :F] = 30.0
    g[1, F:] = 2.0                    # silu(30) = 30 to f32 precision
    g[2, :F] = np.linspace(-4, 4, F, dtype=np.float32)
    g[2, F:] = 1.0
    g[3, :F] = -np.linspace(-4, 4, F, dtype=np.float32)
    g[3, F:] = 1.0
    _, _, _, h = oracle.swiglu_quant(g, F)
    assert np.all(h[0] == 0)
    assert np.allclose(h[1], 60.0, rtol=1e-6)
    z = g[2, :F].astype(np.float64)
    assert np.allclose(h[2], z / (1 + np.exp(-z)), rtol=1e-6, atol=1e-7)
    assert np.allclose(h[2] - h[3], z, rtol=1e-5, atol=1e-6)       # silu(z) - silu(-z) = z
    _, _, _, hg = oracle.swiglu_quant(g, F, gelu=True)
    assert np.allclose(hg[2] - hg[3], z, rtol=1e-5, atol=1e-6)      # gelu(z) - gelu(-z) = z
    ref = 0.5 * z * (1 + np.tanh(0.7978845608 * (z + 0.044715 * z ** 3)))
    assert np.allclose(hg[2], ref, rtol=1e-5, atol=1e-6)
    # fused: the row itself
    rows = np.random.default_rng(2).standard_normal((3, F)).astype(np.float32)
    aq, asc, absum, hf = oracle.swiglu_quant(rows, F, fused=True, M_stride=4)
    assert np.array_equal(hf[:3], rows) and np.all(hf[3] == 0)
    q2, s2, a2 = oracle.quantize_act(rows, M_stride=4)
    assert np.array_equal(q2, aq) and np.array_equal(s2, asc) and np.array_equal(a2, absum)


def test_add_norm_quant_forms():
    rng = np.random.default_rng(3)
    K, eps, s = 1024, 1e-6, 0.75
    x = rng.standard_normal((3, K)).astype(np.float32)
    t = rng.standard_normal((3, K)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    w2 = rng.uniform(0.5, 1.5, K).astype(np.float32)
    # t = 0: x_new = x * s exactly, and without w2 the quantized values are quantize(x_new)
    xn, aq, asc, absum, h = oracle.add_norm_quant(x, np.zeros_like(t), w, eps, s)
    assert np.array_equal(xn, (x * np.float32(s)).astype(np.float32)) and np.array_equal(h, xn)
    q2, s2, _ = oracle.quantize_act(xn)
    assert np.array_equal(q2, aq) and np.array_equal(s2, asc)
    # general case against float64
    xn, aq, asc, absum, h = oracle.add_norm_quant(x, t, w, eps, s, w2=w2, M_stride=4)
    xr = (x.astype(np.float64) + t * f64_rms(t, eps) * w) * s
    assert np.max(np.abs(xn - xr)) / np.max(np.abs(xr)) < 1e-6
    yr = xr * f64_rms(xr, eps) * w2
    assert np.max(np.abs(h[:3] - yr)) / np.max(np.abs(yr)) < 1e-6
    assert np.all(aq[3] == 0) and np.all(asc[:, 3] == 0)
