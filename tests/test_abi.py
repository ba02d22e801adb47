"""The C ABI on the CPU: exports, signatures, status codes, argument
validation and the host-side RoPE tables. Nothing here launches a kernel:
every call below fails validation (or is a zero-size no-op) before the
library touches HIP."""
import ctypes
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

from headshot_amd import _lib, rope
from headshot_amd.parity import assert_bit_exact
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
L = _lib.load()
FAKE = ctypes.c_void_p(0x10000)      # never dereferenced: calls fail validation first
FAKE2 = ctypes.c_void_p(0x20000)


def test_library_exports_every_header_function():
    declared = _lib.header_functions()
    assert len(declared) >= 17
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [f for f in declared if f not in exported]
    assert not missing, f"declared in include/headshot_hip.h but not exported: {missing}"
    for f in declared:
        assert hasattr(L, f)


def test_binding_table_matches_header():
    assert sorted(_lib.SIGNATURES) == _lib.header_functions()


def test_abi_version_and_status_strings():
    assert L.hs_abi_version() == _lib.ABI_VERSION
    for code, name in [(0, b"HS_OK"), (-1, b"HS_EINVAL"), (-2, b"HS_EHIP"), (-3, b"HS_EUNSUPPORTED")]:
        assert L.hs_status_string(code) == name
    assert L.hs_status_string(7) == b"HS_UNKNOWN"


def _einval(status, needle):
    assert status == _lib.HS_EINVAL, _lib.status_name(status)
    msg = L.hs_last_error().decode()
    assert needle in msg, msg


F16, F32 = _lib.HS_F16, _lib.HS_F32


def test_layernorm_contract():
    _einval(L.hs_layernorm(None, 7, FAKE, FAKE, FAKE, FAKE2, 4, 64, 1e-5), "dtype")
    _einval(L.hs_layernorm(None, F16, FAKE, FAKE, FAKE, FAKE2, -1, 64, 1e-5), "rows")
    _einval(L.hs_layernorm(None, F16, FAKE, FAKE, FAKE, FAKE2, 4, 0, 1e-5), "dim")
    _einval(L.hs_layernorm(None, F16, None, FAKE, FAKE, FAKE2, 4, 64, 1e-5), "null")
    # out partially overlapping x (x rows are 128 bytes apart)
    _einval(L.hs_layernorm(None, F16, FAKE, FAKE, FAKE, ctypes.c_void_p(0x10000 + 128), 4, 64,
                           1e-5), "overlap")
    assert L.hs_layernorm(None, F16, None, None, None, None, 0, 64, 1e-5) == _lib.HS_OK


def test_qknorm_rope_contract():
    q = L.hs_qknorm_rope
    _einval(q(None, F16, FAKE, FAKE, None, None, None, FAKE2, 2, 11, 16, 64, 5, 1e-5), "norm weight")
    _einval(q(None, F16, FAKE, None, None, FAKE, None, FAKE2, 2, 11, 16, 64, 5, 1e-5), "sin and cos")
    _einval(q(None, F16, FAKE, None, None, FAKE, FAKE, FAKE2, 2, 11, 16, 64, 12, 1e-5), "prefix")
    _einval(q(None, F16, FAKE, None, None, FAKE, FAKE, FAKE2, 2, 11, 16, 63, 5, 1e-5), "even")
    _einval(q(None, F16, FAKE, None, None, None, None, FAKE, 2, 11, 16, 64, 5, 1e-5), "overlap")
    _einval(q(None, F16, FAKE, None, None, None, None, FAKE2, -2, 11, 16, 64, 5, 1e-5), "negative")
    _einval(q(None, F16, FAKE, None, None, None, None, FAKE2, 1 << 16, 1 << 12, 16, 64, 5, 1e-5),
            "2^31")
    assert q(None, F16, None, None, None, None, None, None, 0, 11, 16, 64, 5, 1e-5) == _lib.HS_OK


def test_qknorm_rope_pair_contract():
    q = L.hs_qknorm_rope_pair
    K, QH, KH = ctypes.c_void_p(0x30000), FAKE2, ctypes.c_void_p(0x40000)
    shape = (2, 11, 16, 64, 5, 1e-5)
    _einval(q(None, 7, FAKE, K, None, None, None, None, None, None, QH, KH, *shape), "dtype")
    _einval(q(None, F16, FAKE, K, FAKE, None, None, None, None, None, QH, KH, *shape),
            "weight and bias")
    _einval(q(None, F16, FAKE, K, FAKE, FAKE, None, None, None, None, QH, KH, *shape),
            "both q and k")
    _einval(q(None, F16, FAKE, K, None, None, None, None, FAKE, None, QH, KH, *shape), "sin and cos")
    _einval(q(None, F16, FAKE, K, None, None, None, None, FAKE, FAKE, QH, KH, 2, 11, 16, 64, 12,
              1e-5), "prefix")
    _einval(q(None, F16, FAKE, K, None, None, None, None, None, None, QH, None, *shape), "null")
    # each output against each input, and the outputs against each other
    _einval(q(None, F16, FAKE, K, None, None, None, None, None, None, QH, K, *shape), "overlaps an input")
    _einval(q(None, F16, FAKE, K, None, None, None, None, None, None, FAKE, KH, *shape),
            "overlaps an input")
    _einval(q(None, F16, FAKE, K, None, None, None, None, None, None, QH, QH, *shape),
            "q_head overlaps k_head")
    assert q(None, F16, None, None, None, None, None, None, None, None, None, None, 0, 11, 16, 64,
             5, 1e-5) == _lib.HS_OK


def test_split_rope_apply_contract():
    _einval(L.hs_split_heads(None, F32, FAKE, FAKE, 2, 5, 4, 8), "overlap")
    _einval(L.hs_split_heads(None, F32, None, FAKE, 2, 5, 4, 8), "null")
    _einval(L.hs_rope_apply(None, F32, FAKE, FAKE, FAKE, 2, 3, 11, 64, 12), "prefix")
    _einval(L.hs_rope_apply(None, F32, FAKE, FAKE, FAKE, 2, 3, 11, 63, 5), "odd")
    _einval(L.hs_rope_apply(None, F32, FAKE, None, FAKE, 2, 3, 11, 64, 5), "null")
    # every token inside the prefix: nothing to rotate
    assert L.hs_rope_apply(None, F32, FAKE, None, None, 2, 3, 11, 64, 11) == _lib.HS_OK


def test_elementwise_contracts():
    _einval(L.hs_bias_gelu(None, F16, FAKE, None, FAKE2, -1, 4096), "rows")
    _einval(L.hs_bias_gelu(None, F16, FAKE, None, ctypes.c_void_p(0x10000 + 2), 2, 4096), "overlap")
    _einval(L.hs_gelu(None, F16, FAKE, FAKE2, -5), "negative")
    _einval(L.hs_bias_ls_residual(None, F16, FAKE, FAKE2, None, None, ctypes.c_void_p(0x30000), 4,
                                  1024), "null")
    _einval(L.hs_residual_ls(None, F16, FAKE, FAKE2, FAKE, ctypes.c_void_p(0x30000), 1000, 300),
            "multiple")
    _einval(L.hs_cast_f32_to_f16(None, FAKE, ctypes.c_void_p(0x10000 + 8), 100), "overlap")
    _einval(L.hs_tiled_add(None, FAKE, FAKE2, FAKE, 10, 3), "tile")
    _einval(L.hs_copy_rows(None, FAKE, 0, ctypes.c_void_p(0x10000 + 64), 0, 4, 128), "overlap")
    assert L.hs_copy_rows(None, None, 0, None, 0, 0, 128) == _lib.HS_OK
    assert L.hs_gelu(None, F16, None, None, 0) == _lib.HS_OK


def test_size_limits():
    """Tensors of 2^40 elements or more are refused before anything is
    launched (byte counts and offsets then stay far inside 64 bits)."""
    big = 1 << 31  # rows; x 1024 columns = 2^41 elements
    _einval(L.hs_layernorm(None, F16, FAKE, FAKE, FAKE, FAKE2, big, 1024, 1e-5), "too large")
    _einval(L.hs_layernorm_stats(None, F16, FAKE, FAKE2, big, 1024, 1e-5), "too large")
    _einval(L.hs_bias_ls_residual_layernorm(None, F16, FAKE, FAKE, None, FAKE, FAKE, FAKE, FAKE2,
                                            FAKE2, big, 1024, 1e-5), "too large")
    _einval(L.hs_bias_gelu(None, F16, FAKE, None, FAKE2, big, 4096), "too large")
    _einval(L.hs_gelu(None, F16, FAKE, FAKE2, 1 << 41), "too large")
    _einval(L.hs_bias_ls_residual(None, F16, FAKE, FAKE, None, FAKE, FAKE2, big, 1024),
            "too large")
    _einval(L.hs_cast_f32_to_f16(None, FAKE, FAKE2, 1 << 40), "too large")
    _einval(L.hs_cast_f16_to_f32(None, FAKE, FAKE2, 1 << 40), "too large")
    _einval(L.hs_tiled_add(None, FAKE, FAKE2, FAKE, 1 << 40, 1024), "too large")
    _einval(L.hs_copy_rows(None, FAKE, 0, FAKE2, 0, 1 << 40, 2048), "too large")
    _einval(L.hs_copy_rows(None, FAKE, 1 << 40, FAKE2, 0, 4, 2048), "too large")
    # just below the limit the checks pass on to the next one (null buffers)
    _einval(L.hs_layernorm(None, F16, None, FAKE, FAKE, FAKE2, (1 << 30) - 1, 1024, 1e-5), "null")


def test_assemble_contract():
    a = L.hs_assemble_tokens
    _einval(a(None, F16, FAKE, F32, None, None, FAKE2, FAKE2, FAKE, 2, 6, 4, 1024, 3), "n_var")
    _einval(a(None, F16, FAKE, F32, None, None, None, FAKE2, ctypes.c_void_p(0x100000), 2, 6, 4,
              1024, 2), "null")
    _einval(a(None, F16, FAKE, 5, None, None, FAKE2, FAKE2, FAKE, 2, 6, 4, 1024, 2), "dtype")
    assert a(None, F16, None, F32, None, None, None, None, None, 0, 6, 4, 1024, 2) == _lib.HS_OK


def test_attention_and_merge_contract():
    a = L.hs_attention
    _einval(a(None, 7, FAKE, FAKE, FAKE, FAKE2, 1, 2, 8, 64), "dtype")
    _einval(a(None, F16, FAKE, FAKE, FAKE, FAKE2, 1, -2, 8, 64), "shape")
    _einval(a(None, F16, None, FAKE, FAKE, FAKE2, 1, 2, 8, 64), "null")
    _einval(a(None, F16, FAKE, FAKE, FAKE, ctypes.c_void_p(0x10000 + 64), 1, 2, 8, 64), "overlap")
    _einval(a(None, F16, FAKE, FAKE, FAKE, FAKE2, 1 << 20, 1 << 10, 4, 64), "2^31")
    # f16 with head_dim 128, or head_dim 32: the reference has no such variant
    big = [ctypes.c_void_p(0x1000000 * i) for i in range(1, 5)]
    assert a(None, F16, *big, 1, 2, 8, 128) == _lib.HS_EUNSUPPORTED
    assert a(None, F32, *big, 1, 2, 8, 32) == _lib.HS_EUNSUPPORTED
    assert L.hs_attention_merged(None, F32, *big, 1, 2, 8, 48) == _lib.HS_EUNSUPPORTED
    assert a(None, F16, None, None, None, None, 0, 2, 8, 64) == _lib.HS_OK
    m = L.hs_attn_merge
    _einval(m(None, F16, None, FAKE2, 1, 2, 8, 64), "null")
    _einval(m(None, F16, FAKE, ctypes.c_void_p(0x10000 + 16), 1, 2, 8, 64), "overlap")
    assert m(None, F16, None, None, 0, 2, 8, 64) == _lib.HS_OK


def test_cache_and_row_block_contract():
    _einval(L.hs_concat_channels(None, 9, FAKE, FAKE, FAKE2, 4, 8, 8), "dtype")
    _einval(L.hs_concat_channels(None, F16, None, FAKE, FAKE2, 4, 8, 8), "null")
    _einval(L.hs_cache_build(None, F16, FAKE, FAKE, ctypes.c_void_p(0x10000 + 32), 4, 8, 8),
            "overlap")
    assert L.hs_cache_build(None, F16, None, None, None, 0, 8, 8) == _lib.HS_OK
    _einval(L.hs_cast_f16_to_f32(None, FAKE, None, 8), "null")
    _einval(L.hs_cast_f16_to_f32(None, FAKE, FAKE, -1), "negative")
    r = L.hs_copy_row_blocks
    _einval(r(None, FAKE, 0, 2, ctypes.c_void_p(0x1000000), 0, 4, 5, 3, 64), "stride")
    _einval(r(None, FAKE, 0, 4, ctypes.c_void_p(0x10000 + 64), 0, 4, 5, 2, 64), "overlap")
    _einval(r(None, FAKE, -1, 4, FAKE2, 0, 4, 5, 2, 64), "negative")
    assert r(None, None, 0, 4, None, 0, 4, 0, 2, 64) == _lib.HS_OK


def test_linear_contract():
    big = [ctypes.c_void_p(0x1000000 * i) for i in range(1, 6)]
    _einval(L.hs_linear(None, 4, big[0], big[1], None, big[2], 4, 128, 64), "dtype")
    _einval(L.hs_linear(None, F16, big[0], big[1], None, big[2], -4, 128, 64), "shape")
    _einval(L.hs_linear(None, F16, None, big[1], None, big[2], 4, 128, 64), "null")
    _einval(L.hs_linear(None, F16, big[0], big[1], None, ctypes.c_void_p(0x1000000 + 64), 4, 128, 64),
            "overlap")
    _einval(L.hs_linear_gelu(None, F16, big[0], None, None, big[2], 4, 128, 64), "null")
    _einval(L.hs_linear_ls_residual(None, F16, big[0], big[1], None, None, big[3], big[2], 4, 128, 64),
            "gamma")
    _einval(L.hs_linear_ls_residual(None, F16, big[0], big[1], None, big[4], None, big[2], 4, 128, 64),
            "null")
    # out partly over res (equal is allowed: in place)
    _einval(L.hs_linear_ls_residual(None, F16, big[0], big[1], None, big[4], big[3],
                                    ctypes.c_void_p(0x4000000 + 2), 4, 128, 64), "res")
    assert L.hs_linear(None, F16, None, None, None, None, 0, 128, 64) == _lib.HS_OK


def test_linear_qkv_heads_contract():
    """Validation before any launch: fake, non-overlapping device addresses
    (x, w, q, k, v at 16 MiB steps, each region far larger than its use)."""
    x, w, q, k, v = (ctypes.c_void_p(0x1000000 * i) for i in range(1, 6))
    nw = nb = ctypes.c_void_p(0x9000000)
    f = L.hs_linear_qkv_heads

    def call(dt=F16, x=x, w=w, qw=nw, qb=nb, kw=nw, kb=nb, sn=None, cs=None, q=q, k=k, v=v,
             S=2, T=8, H=4, d=64, kk=64, prefix=0, eps=1e-5):
        return f(None, dt, x, w, None, qw, qb, kw, kb, sn, cs, q, k, v, S, T, H, d, kk, prefix, eps)

    assert call() is not None  # signature binds
    _einval(call(dt=4), "dtype")
    _einval(call(H=0), "shape")
    _einval(call(prefix=9), "prefix")
    _einval(call(qb=None), "weight and bias")
    _einval(call(sn=nw), "both tables")
    _einval(call(eps=0.0), "eps")
    _einval(call(k=None), "null")
    _einval(call(x=None), "null")
    _einval(call(k=ctypes.c_void_p(0x3000000 + 64)), "outputs overlap")
    _einval(call(v=ctypes.c_void_p(0x1000000 + 64)), "overlaps x or w")
    # f32 with an odd H (3 * 3 * 64 = 576 columns, not whole 128-column tiles)
    assert call(dt=_lib.HS_F32, H=3) == _lib.HS_EUNSUPPORTED
    # each output is (S*T, H*d), not (S*T, 3*H*d): w may start right after q
    # (that f32 shape stops with HS_EUNSUPPORTED after the overlap checks,
    # before any launch)
    assert call(dt=_lib.HS_F32, H=3,
                w=ctypes.c_void_p(0x3000000 + 2 * 8 * 3 * 64 * 4)) == _lib.HS_EUNSUPPORTED
    assert call(dt=_lib.HS_F32, kk=48) == _lib.HS_EUNSUPPORTED  # f32 k stages of 32
    assert call(d=32) == _lib.HS_EUNSUPPORTED
    assert call(H=2) == _lib.HS_EUNSUPPORTED            # 3 * 2 * 64 = 384 columns
    assert call(S=0) == _lib.HS_OK                      # zero tokens: no-op


def test_python_surface_raises_contract_errors():
    with pytest.raises(_lib.HsContractError) as e:
        _lib.check(L.hs_gelu(None, F16, FAKE, FAKE2, -5), "gelu")
    assert isinstance(e.value, AssertionError)


# ------------------------------------------------------------ host RoPE tables

def test_periods_bit_exact():
    assert_bit_exact(rope.periods(), O.rope_periods(), "periods vs oracle")
    g = json.load(open(os.path.join(HERE, "golden", "rope_tables.json")))
    assert [f"{v:08x}" for v in rope.periods().view(np.uint32)] == g["periods_bits"]


def test_tables_bit_exact_against_golden_and_oracle():
    g = json.load(open(os.path.join(HERE, "golden", "rope_tables.json")))
    per = rope.periods()
    for name, fx in g["grids"].items():
        sin, cos = rope.tables(per, fx["h_p"], fx["w_p"])
        assert hashlib.sha256(sin.tobytes()).hexdigest() == fx["sin_sha256"], name
        assert hashlib.sha256(cos.tobytes()).hexdigest() == fx["cos_sha256"], name
        osin, ocos = O.rope_tables(per, fx["h_p"], fx["w_p"])
        assert_bit_exact(sin, osin, f"sin {name}")
        assert_bit_exact(cos, ocos, f"cos {name}")


def test_tables_position_mapping_non_square():
    """Rows are h-outer / w-inner (engine/rope.rs:27-29): row r*w_p + c has its
    h-angles from r and its w-angles from c."""
    per = rope.periods()
    sin, cos = rope.tables(per, 21, 37)
    col = rope.tables(per, 37, 37)[0]  # same side length, so same coordinates
    for r, c in [(0, 0), (3, 17), (20, 36), (10, 0)]:
        row = r * 37 + c
        assert_bit_exact(sin[row, :16], col[r * 37, :16], "h-angles follow the row")
        assert_bit_exact(sin[row, 16:32], col[c, 16:32], "w-angles follow the column")


def test_tables_contract():
    s = np.empty((6, 64), np.float32)
    st = L.hs_rope_tables(None, 2, 3, s.ctypes.data, s.ctypes.data)
    _einval(st, "null")
    _einval(L.hs_rope_tables(rope.periods().ctypes.data, -1, 3, s.ctypes.data, s.ctypes.data),
            "negative")
    assert L.hs_rope_tables(None, 0, 3, None, None) == _lib.HS_OK
