"""Pins the CPU oracle (oracle/hs_oracle.c) before it is trusted as checker.

Each oracle function is checked against something that does not share its
code: the reference's own unit-test values and tolerances (re-expressed
here with the same seeds), independent libraries (numpy float16 rounding,
float64 torch layer_norm, math.erf), closed forms and invariants, and brute
force. The cases are chosen so that a plausible slip (dropped eps, wrong
sign in the rotation, swapped table halves, transposed operands, a missing
storage rounding) fails at least one of them.
"""
import hashlib
import json
import math
import os

import numpy as np
import pytest
import torch

from headshot_amd.parity import assert_bit_exact, assert_close
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))


# ------------------------------------------------------------------ inputs

def _splitmix_py(seed, n, denom, last_xor=True):
    """SplitMix64 in plain Python ints (tests/kernels.rs:7-23; with
    ``last_xor=False`` the variant of tests/dense_kernels.rs:6-17, which
    stops before ``z ^= z >> 31``)."""
    out, state = [], seed
    mask = (1 << 64) - 1
    for _ in range(n):
        state = (state + 0x9E3779B97F4A7C15) & mask
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        if last_xor:
            z ^= z >> 31
        v = np.float32(z >> 40) / np.float32(denom)
        out.append(np.float32(np.float32(v * np.float32(2.0)) - np.float32(1.0)))
    return np.array(out, np.float32)


def test_rng_matches_reference_splitmix():
    assert_bit_exact(O.rng_vec(3, 257), _splitmix_py(3, 257, 1 << 23), "Rng(3)")
    assert_bit_exact(O.rng_vec(4, 100), _splitmix_py(4, 100, 1 << 23), "Rng(4)")
    v = O.rng_vec(3, 10000)
    assert v.min() >= -1.0 and v.max() < 3.0  # the reference's scaling spans [-1, 3)
    r = O.rvec_f16(7, 1000)
    want = _splitmix_py(7, 1000, 1 << 24).astype(np.float16).astype(np.float32)
    assert_bit_exact(r, want, "rvec f16")
    d = O.rvec(2, 120)
    assert_bit_exact(d, _splitmix_py(2, 120, 1 << 24, last_xor=False), "dense rvec")
    assert d.min() >= -1.0 and d.max() < 1.0


def test_normal_is_seeded_standard_normal():
    a = O.normal(42, (200000,))
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1.0) < 0.01
    assert_bit_exact(a, O.normal(42, (200000,)), "normal determinism")


# --------------------------------------------------------------- f16 storage

def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(0)
    scales = rng.choice(np.array([1e-9, 1e-7, 6e-5, 1e-3, 1.0, 300.0, 6e4, 7e4], np.float32), 400000)
    x = (rng.standard_normal(400000).astype(np.float32) * scales).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 6.1035156e-05,
                      6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 8.940697e-08,
                      np.inf, -np.inf, 1.0009766, 1.0004883, 1.0014648], np.float32)
    x = np.concatenate([x, edges, np.nextafter(edges, np.float32(np.inf))]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16)
    assert_bit_exact(O.to_f16(x), want, "f32->f16")
    h = np.arange(65536, dtype=np.uint16).view(np.float16)
    h = h[~np.isnan(h)]
    assert_bit_exact(O.f16_to_f32(h), h.astype(np.float32), "f16->f32 (all non-nan)")


# ---------------------------------------------------------------- RoPE tables

def test_periods_reference_values():
    p = O.rope_periods()
    # engine/rope.rs:61-67
    assert p[0] == 1.0
    assert abs(p[8] - 10.0) < 1e-4
    assert abs(p[15] - np.float32(100.0) ** np.float32(30.0 / 32.0)) < 1e-3
    # each is the correctly rounded value of 100^(2i/32)
    for i in range(16):
        e = np.float32(np.float32(2 * i) / np.float32(32))
        assert p[i] == np.float32(100.0 ** float(e)), i


def test_tables_reference_closed_forms():
    # engine/rope.rs:69-90 (2x3 grid)
    sin, cos = O.rope_tables(O.rope_periods(), 2, 3)
    assert sin.shape == (6, 64)
    angle = np.float32(2 * math.pi) * (np.float32(2.0) * (np.float32(2.5) / np.float32(3.0)) - np.float32(1.0))
    idx = 5
    assert abs(sin[idx, 16] - math.sin(angle)) < 1e-6
    assert abs(cos[idx, 16] - math.cos(angle)) < 1e-6
    assert abs(sin[idx, 0]) < 1e-6 and abs(cos[idx, 0] - 1.0) < 1e-6
    for j in range(32):
        assert sin[idx, j] == sin[idx, 32 + j] and cos[idx, j] == cos[idx, 32 + j]
    # short axis does not span [-1, 1] on a non-square grid (coords over max side)
    sin, cos = O.rope_tables(O.rope_periods(), 21, 37)
    ang_h0 = math.atan2(sin[0, 0], cos[0, 0])
    want = 2 * math.pi * (2 * (0.5 / 37) - 1)
    assert abs(math.remainder(ang_h0 - want, 2 * math.pi)) < 1e-5


@pytest.mark.parametrize("grid", [(2, 3), (37, 37), (21, 37), (37, 21), (4, 4)])
def test_tables_vs_correctly_rounded_sin_cos(grid):
    """Rebuild every angle with numpy f32 arithmetic (the reference's operand
    order) and compare the oracle's sin/cos with the correctly rounded f32 of
    the exact sin/cos of that angle. glibc's sinf/cosf are within 1 ulp; an
    index or channel mix-up would be far off."""
    h_p, w_p = grid
    per = O.rope_periods()
    sin, cos = O.rope_tables(per, h_p, w_p)
    side = np.float32(max(h_p, w_p))
    tau = np.float32(6.28318530717958647692)
    coord = lambda i: np.float32(2.0) * ((np.float32(i) + np.float32(0.5)) / side) - np.float32(1.0)  # noqa: E731
    worst = 0
    for r in range(h_p):
        for c in range(w_p):
            row = r * w_p + c
            for i in range(16):
                for off, ci in ((0, coord(r)), (16, coord(c))):
                    a = np.float32(np.float32(tau * ci) / per[i])
                    for half in (0, 32):
                        s_cr = np.float32(math.sin(float(a)))
                        c_cr = np.float32(math.cos(float(a)))
                        s_o, c_o = sin[row, half + off + i], cos[row, half + off + i]
                        for got, cr in ((s_o, s_cr), (c_o, c_cr)):
                            d = abs(int(np.array(got).view(np.int32)) - int(np.array(cr).view(np.int32)))
                            worst = max(worst, d)
    assert worst <= 1, f"max ulp distance {worst}"


def test_tables_match_golden_fixtures():
    g = json.load(open(os.path.join(HERE, "golden", "rope_tables.json")))
    per = O.rope_periods()
    assert [f"{v:08x}" for v in per.view(np.uint32)] == g["periods_bits"]
    for name, fx in g["grids"].items():
        sin, cos = O.rope_tables(per, fx["h_p"], fx["w_p"])
        assert hashlib.sha256(sin.tobytes()).hexdigest() == fx["sin_sha256"], name
        assert hashlib.sha256(cos.tobytes()).hexdigest() == fx["cos_sha256"], name
        for r, rowfx in fx["rows"].items():
            assert [f"{v:08x}" for v in sin[int(r)].view(np.uint32)] == rowfx["sin"], (name, r)
            assert [f"{v:08x}" for v in cos[int(r)].view(np.uint32)] == rowfx["cos"], (name, r)


# ------------------------------------------------------------------ RoPE apply

def test_rope_apply_cpu_is_complex_rotation():
    sin, cos = O.rope_tables(O.rope_periods(), 4, 4)
    x = np.array([math.sin(i * 0.37) for i in range(64)], np.float32)
    for row in (0, 7, 15):
        y = O.rope_apply_cpu(x, sin, cos, row).astype(np.float64)
        theta = np.arctan2(sin[row, :32].astype(np.float64), cos[row, :32].astype(np.float64))
        z = (x[:32] + 1j * x[32:].astype(np.float64)) * np.exp(1j * theta)
        np.testing.assert_allclose(y[:32], z.real, atol=2e-6)
        np.testing.assert_allclose(y[32:], z.imag, atol=2e-6)
        # engine/rope.rs:92-103: pair norms preserved
        before = np.hypot(x[:32], x[32:])
        after = np.hypot(y[:32], y[32:])
        assert np.abs(before - after).max() < 1e-5


def test_rope_apply_matches_cpu_reference_test():
    """tests/kernels.rs:149-182: (S,H,T,D) = (2,3,11,64), prefix 5, 2x3 grid, Rng(4)."""
    s, h, t, d, prefix = 2, 3, 11, 64, 5
    sin, cos = O.rope_tables(O.rope_periods(), 2, 3)
    x = O.rng_vec(4, s * h * t * d).reshape(s, h, t, d)
    got = O.rope_apply(x, sin, cos, prefix)
    for si in range(s):
        for hi in range(h):
            for ti in range(t):
                want = x[si, hi, ti] if ti < prefix else O.rope_apply_cpu(x[si, hi, ti], sin, cos, ti - prefix)
                assert_close(got[si, hi, ti], want, 1e-5, "rope")
    # sign of the rotation: an independent complex-number restatement
    theta = np.arctan2(sin[:, :32].astype(np.float64), cos[:, :32].astype(np.float64))
    z = (x[..., prefix:, :32] + 1j * x[..., prefix:, 32:].astype(np.float64)) * np.exp(1j * theta)
    np.testing.assert_allclose(got[..., prefix:, :32], z.real, atol=1e-5)
    np.testing.assert_allclose(got[..., prefix:, 32:], z.imag, atol=1e-5)


# ------------------------------------------------------------------ LayerNorm

def _torch_ln(x, w, b, eps):
    xt = torch.from_numpy(np.asarray(x, np.float64))
    return torch.nn.functional.layer_norm(xt, (xt.shape[-1],), torch.from_numpy(np.asarray(w, np.float64)),
                                          torch.from_numpy(np.asarray(b, np.float64)), eps).numpy()


def test_layernorm_matches_cpu_reference_test():
    """tests/kernels.rs:100-126: rows 19, dim 300, Rng(3), tol 1e-4."""
    rows, dim = 19, 300
    rng = O.rng_vec(3, rows * dim + 2 * dim)
    x = rng[: rows * dim].reshape(rows, dim)
    w, b = rng[rows * dim: rows * dim + dim], rng[rows * dim + dim:]
    got = O.layernorm(x, w, b, 1e-5)
    assert_close(got, _torch_ln(x, w, b, 1e-5), 1e-4, "layernorm")


@pytest.mark.parametrize("dim", [64, 300, 1024, 4096])
@pytest.mark.parametrize("scale", [1.0, 1e-3])
@pytest.mark.parametrize("eps", [1e-5, 1e-6])
def test_layernorm_vs_float64_library(dim, scale, eps):
    # scale 1e-3 gives variance ~1e-6, where eps matters: a dropped or
    # misplaced eps fails this
    x = ((O.normal(5, (23, dim)) + np.float32(0.3)) * np.float32(scale)).astype(np.float32)
    w, b = O.normal(6, (dim,), 1.0, 0.5), O.normal(7, (dim,), 0.0, 0.5)
    assert_close(O.layernorm(x, w, b, eps), _torch_ln(x, w, b, eps), 1e-5, f"layernorm {dim}")


def test_layernorm_f16_storage_rounding():
    x16 = O.to_f16(O.normal(8, (17, 1024)))
    w, b = O.normal(9, (1024,), 1.0, 0.02), O.normal(10, (1024,), 0.0, 0.02)
    got = O.layernorm(x16, w, b, 1e-6)
    f32 = O.layernorm(x16.astype(np.float32), w, b, 1e-6)
    assert_bit_exact(got, f32.astype(np.float16), "f16 LN == round(f32 LN of f16 input)")


# ----------------------------------------------------------------------- GELU

def test_gelu_matches_erf_reference_test():
    """tests/kernels.rs:128-147: x = -8..8 step 0.2 vs f64 erf, |err| < 1e-5."""
    xs = np.array([i * 0.2 for i in range(-40, 41)], np.float32)
    got = O.gelu(xs)
    for x, g in zip(xs, got):
        exact = 0.5 * float(x) * (1.0 + math.erf(float(x) / math.sqrt(2.0)))
        assert abs(float(g) - exact) < 1e-5, (x, g, exact)
    assert O.gelu(np.array([0.0], np.float32))[0] == 0.0
    assert abs(O.gelu(np.array([10.0], np.float32))[0] - 10.0) < 1e-6
    assert abs(O.gelu(np.array([-10.0], np.float32))[0]) < 1e-6


def test_erf_as_published_accuracy():
    # A&S 7.1.26: |error| <= 1.5e-7 (plus f32 evaluation noise)
    for v in np.linspace(-4, 4, 2001, dtype=np.float32):
        assert abs(O.erf_as(float(v)) - math.erf(float(v))) < 5e-7, v
    assert O.erf_as(0.5) > 0 > O.erf_as(-0.5)


def test_gelu_f16_storage_rounding():
    x = O.rvec_f16(1, 4096).astype(np.float16)
    assert_bit_exact(O.gelu(x), O.gelu(x.astype(np.float32)).astype(np.float16), "f16 gelu")


# ------------------------------------------------------- layout and residual

def test_split_heads_merge_roundtrip_reference_test():
    """tests/kernels.rs:241-274: (s,t,h,d) = (2,5,4,8), Rng(6), exact."""
    s, t, h, d = 2, 5, 4, 8
    x = O.rng_vec(6, s * t * h * d).reshape(s * t, h * d)
    q = O.split_heads(x, s, t, h, d)
    assert_bit_exact(q, np.ascontiguousarray(x.reshape(s, t, h, d).transpose(0, 2, 1, 3)), "split")
    assert_bit_exact(O.attn_merge(q), x, "merge")
    x16 = x.astype(np.float16)
    assert_bit_exact(O.split_heads(x16, s, t, h, d),
                     np.ascontiguousarray(x16.reshape(s, t, h, d).transpose(0, 2, 1, 3)), "split f16")


@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_residual_bias_cast_tiled_add(dt):
    res = O.to_f16(O.normal(11, (9, 300))) if dt == np.float16 else O.normal(11, (9, 300))
    x = O.to_f16(O.normal(12, (9, 300))) if dt == np.float16 else O.normal(12, (9, 300))
    g, b = O.normal(13, (300,)), O.normal(14, (300,), 0, 0.02)
    want = (res.astype(np.float32) + (g[None, :] * x.astype(np.float32)).astype(np.float32)).astype(dt)
    assert_bit_exact(O.residual_ls(res, x, g), want, "residual_ls")
    assert_bit_exact(O.add_bias(x, b), (x.astype(np.float32) + b).astype(dt), "add_bias")
    f = O.normal(15, (3, 7, 5))
    assert_bit_exact(O.cast_to_f16(f), f.astype(np.float16), "cast")
    tab = O.normal(16, (7, 5))
    assert_bit_exact(O.tiled_add(f, tab), (f + tab[None]).astype(np.float32), "tiled_add")


def test_every_op_f16_matches_f32_reference_test():
    """tests/f16_ops.rs:36-109 on the oracle: (S,H,T,D) = (2,4,21,64) with
    f16-exact inputs; max-abs tolerances as in the reference."""
    s, h, t, d = 2, 4, 21, 64
    c, rows = h * d, s * t
    x = O.rvec_f16(1, rows * c).reshape(rows, c)
    x16 = x.astype(np.float16)
    w, b = O.rvec_f16(2, c), O.rvec_f16(3, c)
    assert np.abs(O.layernorm(x16, w, b).astype(np.float32) - O.layernorm(x, w, b)).max() < 2e-2
    assert np.abs(O.gelu(x16).astype(np.float32) - O.gelu(x)).max() < 2e-3
    r, g = O.rvec_f16(4, rows * c).reshape(rows, c), O.rvec_f16(5, c)
    assert np.abs(O.residual_ls(r.astype(np.float16), x16, g).astype(np.float32)
                  - O.residual_ls(r, x, g)).max() < 2e-3
    sin, cos = O.rope_tables(O.rope_periods(), 4, 4)
    q = O.rvec_f16(7, s * h * t * d).reshape(s, h, t, d)
    prefix = t - 16
    assert np.abs(O.rope_apply(q.astype(np.float16), sin, cos, prefix).astype(np.float32)
                  - O.rope_apply(q, sin, cos, prefix)).max() < 2e-3


# -------------------------------------------------------------- composites

@pytest.mark.parametrize("dt", [np.float32, np.float16])
@pytest.mark.parametrize("norm,rope", [(True, True), (True, False), (False, True)])
def test_qknorm_rope_composite_is_reference_sequence(dt, norm, rope):
    s, t, h, d, prefix = 2, 11, 3, 64, 5
    x = O.normal(21, (s * t, h * d)).astype(dt)
    nw, nb = O.normal(22, (d,), 1.0, 0.02), O.normal(23, (d,), 0.0, 0.02)
    sin, cos = O.rope_tables(O.rope_periods(), 2, 3)
    seq = O.split_heads(x, s, t, h, d)
    if norm:
        seq = O.layernorm(seq, nw, nb, 1e-6)
    if rope:
        seq = O.rope_apply(seq, sin, cos, prefix)
    got = O.qknorm_rope(x, nw if norm else None, nb if norm else None, sin if rope else None,
                        cos if rope else None, s, t, h, d, prefix, 1e-6)
    assert_bit_exact(got, seq, "qknorm_rope composite")


@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_bias_composites_are_reference_sequence(dt):
    x = O.normal(31, (7, 40)).astype(dt)
    res = O.normal(32, (7, 40)).astype(dt)
    b, g = O.normal(33, (40,), 0, 0.02), O.normal(34, (40,))
    assert_bit_exact(O.bias_gelu(x, b), O.gelu(O.add_bias(x, b)), "bias_gelu")
    assert_bit_exact(O.bias_gelu(x, None), O.gelu(x), "gelu")
    # single-rounding variant: gelu of the f32 sum, rounded once
    xs = x.astype(np.float32) + b
    want = O.gelu(xs).astype(dt) if dt == np.float16 else O.gelu(xs)
    assert_bit_exact(O.bias_gelu(x, b, round_bias=False), want, "bias_gelu single rounding")
    assert_bit_exact(O.bias_ls_residual(res, x, b, g), O.residual_ls(res, O.add_bias(x, b), g), "ls")


@pytest.mark.parametrize("out_dt", [np.float32, np.float16])
@pytest.mark.parametrize("n_var", [1, 2])
def test_assemble_tokens_vs_numpy(out_dt, n_var):
    s, p, r, d = 3, 6, 4, 32
    patches = O.normal(41, (s * p, d))
    pb, pos = O.normal(42, (d,), 0, 0.02), O.normal(43, (p, d), 0, 0.02)
    cam = O.normal(44, (n_var, d)).astype(out_dt)
    reg = O.normal(45, (n_var * r, d)).astype(out_dt)
    got = O.assemble_tokens(patches, pb, pos, cam, reg, s, p, r, out_dt, n_var)
    rows = []
    for f in range(s):
        v = 1 if (n_var == 2 and f) else 0
        rows.append(cam[v:v + 1])
        rows.append(reg[v * r:(v + 1) * r])
        rows.append(((patches[f * p:(f + 1) * p] + pb[None]) + pos).astype(out_dt))
    assert_bit_exact(got, np.concatenate(rows), "assemble")


# --------------------------------------------------------------- attention

def _naive_attention64(q, k, v):
    """The reference test's form (tests/kernels.rs:207-231) in float64: full
    score matrix, max-subtracted exp, normalised weighted sum."""
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    s = np.matmul(q, np.swapaxes(k, -1, -2)) / np.sqrt(q.shape[-1])
    p = np.exp(s - s.max(-1, keepdims=True))
    return np.matmul(p / p.sum(-1, keepdims=True), v)


@pytest.mark.parametrize("t", [17, 64, 150])
def test_attention_matches_cpu_reference_test(t):
    """tests/kernels.rs:185-238: (s, h, d) = (2, 3, 64), Rng(5 + t), 1e-4."""
    s, h, d = 2, 3, 64
    # the reference draws q, k, v from one Rng stream in sequence
    stream = O.rng_vec(5 + t, 3 * s * h * t * d).reshape(3, s, h, t, d)
    q, k, v = stream[0], stream[1], stream[2]
    got = O.attention(q, k, v)
    want = _naive_attention64(q, k, v)
    assert np.abs(got - want).max() < 1e-4
    assert_close(got, want.astype(np.float32), 1e-5, f"attention t={t}")


@pytest.mark.parametrize("d", [64, 128])
def test_attention_invariants(d):
    rng = np.random.default_rng(d)
    s, h, t = 2, 2, 37
    q, k, v = (rng.standard_normal((s, h, t, d)).astype(np.float32) for _ in range(3))
    # constant value rows: every output row is that constant
    vc = np.broadcast_to(rng.standard_normal((s, h, 1, d)).astype(np.float32), v.shape).copy()
    assert_close(O.attention(q, k, vc), vc, 1e-6, "constant V")
    # q = 0: uniform weights, the mean of V over keys
    zq = np.zeros_like(q)
    mean = np.broadcast_to(v.astype(np.float64).mean(2, keepdims=True), v.shape)
    assert_close(O.attention(zq, k, v), mean.astype(np.float32), 1e-5, "q = 0")
    # permuting the keys (k and v rows together) leaves the output unchanged
    perm = rng.permutation(t)
    assert_close(O.attention(q, k[:, :, perm], v[:, :, perm]), O.attention(q, k, v), 1e-5,
                 "key permutation")
    # one key: the output is that key's value row
    assert_bit_exact(O.attention(q[:, :, :1], k[:, :, :1], v[:, :, :1]), v[:, :, :1], "T = 1")
    # the scale is 1/sqrt(D): doubling q is the same as scaling scores by 2
    got = O.attention(2 * q, k, v)
    assert_close(got, _naive_attention64(2 * q, k, v).astype(np.float32), 1e-5, "scale")


def test_attention_f16_storage_and_subset():
    rng = np.random.default_rng(9)
    q, k, v = (O.to_f16(rng.standard_normal((1, 2, 33, 64))) for _ in range(3))
    got = O.attention(q, k, v)
    want = _naive_attention64(q, k, v)
    assert got.dtype == np.float16
    assert_bit_exact(got, O.attention(q.astype(np.float32), k.astype(np.float32),
                                      v.astype(np.float32)).astype(np.float16), "f16 = f32 math, RNE")
    assert np.abs(got.astype(np.float64) - want).max() < 2e-3
    idx = np.array([0, 5, 32], np.int32)
    assert_bit_exact(O.attention(q, k, v, q_idx=idx), got[:, :, idx], "query subset")


# ------------------------------------------------------------- cache build

@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_concat_cast_cache_build_vs_numpy(dt):
    rng = np.random.default_rng(31)
    a = rng.standard_normal((37, 24)).astype(dt)
    b = rng.standard_normal((37, 40)).astype(dt)
    cat = np.concatenate([a, b], axis=1)
    assert_bit_exact(O.concat_channels(a, b), cat, "concat")
    assert_bit_exact(O.cache_build(a, b), cat.astype(np.float32), "cache_build")
    if dt == np.float16:
        x = np.arange(65536, dtype=np.uint16).view(np.float16)
        got = O.cast_to_f32(x)
        want = x.astype(np.float32)
        assert np.array_equal(got.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)])
        assert np.isnan(got[np.isnan(want)]).all()


# ------------------------------------------------------------------ linear

@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_linear_vs_float64_and_exact_integers(dt):
    rng = np.random.default_rng(41)
    x = rng.standard_normal((37, 80)).astype(dt)
    w = rng.standard_normal((48, 80)).astype(dt)
    b = rng.standard_normal(48).astype(np.float32)
    got = O.linear(x, w, b).astype(np.float64)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    tol = 1e-5 if dt == np.float32 else 2e-3
    assert np.all(np.abs(got - want) <= tol * np.maximum(1.0, np.abs(want)) * (4 if dt == np.float32 else 1))
    # small integers: every product and partial sum is exact, so the result is
    xi = rng.integers(-3, 4, (19, 64)).astype(dt)
    wi = rng.integers(-3, 4, (16, 64)).astype(dt)
    assert_bit_exact(O.linear(xi, wi).astype(np.float64), xi.astype(np.float64) @ wi.astype(np.float64).T,
                     "integer linear")
    # row subset
    rows = np.array([0, 5, 36])
    assert_bit_exact(O.linear(x, w, b, rows), O.linear(x, w, b)[rows], "row subset")
