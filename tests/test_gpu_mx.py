"""The matrix-core split kernel (groups of 4 query heads; 4-bit rows at head_dim 64 / 128 / 256, 2-bit rows
at head_dim 128).

It forms every product from exact float16 hi/lo splits and sums in float32, so
it must agree with the float32-product kernel (TQ_F32_PRODUCTS) to float32
rounding on the same inputs, and both must sit at float32 distance from a
float64 decode of the same codes (the oracle's ``decode_packed_reference``,
which restates mlx_ops.py:571-595).  Cases cover the tile edges (1, 15, 16,
17 rows; a split's last, partial tile), several splits, both query dtypes,
GQA groups of 4 and 8 (two head groups per KV head), rotation flags, the
current-token path and large score ranges (lazy rescaling).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torque_oracle as o

pytestmark = pytest.mark.gpu


def _case(seed, *, layers, kv_heads, group, head_dim, seq_len, capacity, q_dtype, q_scale, dev, bits=4):
    rng = np.random.default_rng(seed)
    words = head_dim * bits // 32
    shape = (layers, kv_heads, capacity, words)
    k_codes = rng.integers(0, 2**32, size=shape, dtype=np.uint64).astype(np.uint32)
    v_codes = rng.integers(0, 2**32, size=shape, dtype=np.uint64).astype(np.uint32)
    # distinct key and value codebooks with different power-of-two scales
    k_cent = np.sort(rng.normal(size=1 << bits)).astype(np.float32) * np.float32(1.7)
    v_cent = np.sort(rng.normal(size=1 << bits)).astype(np.float32) * np.float32(0.05)
    q = (rng.normal(size=(layers, kv_heads * group, head_dim)) * q_scale).astype(np.float32)
    q = q.astype(np.float16).astype(np.float32) if q_dtype == torch.float16 else q
    signs_l, signs_r = o.rotation_signs_from_seed(head_dim, seed)
    t = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev) if dt is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev, dt)
    return dict(
        np=dict(k_codes=k_codes, v_codes=v_codes, k_cent=k_cent, v_cent=v_cent, q=q, signs=(signs_l, signs_r)),
        dev=dict(
            query=t(q).to(q_dtype),
            key_codes=t(k_codes.view(np.int32)),
            value_codes=t(v_codes.view(np.int32)),
            key_centroids=t(k_cent),
            value_centroids=t(v_cent),
            signs_left=t(signs_l.astype(np.float32)),
            signs_right=t(signs_r.astype(np.float32)),
        ),
    )


def _decode(c, *, layers, kv_heads, group, head_dim, seq_len, capacity, f32_products, n_splits=None,
            rotate=False, current=None, bits=4):
    from torque_hip.ops import packed_decode

    d = c["dev"]
    return packed_decode(
        d["query"], num_layers=layers, query_heads=kv_heads * group, kv_heads=kv_heads, head_dim=head_dim,
        bit_width=bits, key_codes=d["key_codes"], value_codes=d["value_codes"], capacity=capacity, seq_len=seq_len,
        key_centroids=d["key_centroids"], value_centroids=d["value_centroids"], signs_left=d["signs_left"],
        signs_right=d["signs_right"], rotate_query=rotate, inverse_output=rotate,
        current_keys=None if current is None else current[0], current_values=None if current is None else current[1],
        n_splits=n_splits, f32_products=f32_products, matrix_products=not f32_products,
    ).cpu().numpy()


def _float64_reference(c, *, layers, kv_heads, group, head_dim, seq_len, bits=4):
    """out[L, Hq, D] of the unrotated decode (flags 0), computed in float64 by the oracle."""
    n = c["np"]
    kv = np.arange(kv_heads * group) // group
    out = np.empty((layers, kv_heads * group, head_dim), np.float64)
    for layer in range(layers):
        kc = n["k_codes"][layer][kv][:, :seq_len]
        vc = n["v_codes"][layer][kv][:, :seq_len]
        out[layer] = o.decode_packed_reference(n["q"][layer], kc, vc, n["k_cent"], n["v_cent"], bit_width=bits,
                                               head_dim=head_dim)
    return out


CASES = [
    # (bits, head_dim, kv_heads, group, seq_len, n_splits)
    (4, 128, 2, 4, 1, None),
    (4, 128, 2, 4, 15, None),
    (4, 128, 2, 4, 16, None),
    (4, 128, 2, 4, 17, 1),
    (4, 128, 3, 4, 300, None),
    (4, 128, 2, 8, 5000, None),
    (4, 128, 1, 4, 5000, 7),
    (4, 64, 2, 4, 17, None),
    (4, 64, 4, 4, 2100, None),
    (4, 64, 2, 8, 4097, 3),
    (4, 256, 2, 4, 1, None),
    (4, 256, 2, 4, 17, None),
    (4, 256, 1, 4, 3000, None),
    (4, 256, 2, 4, 5000, 7),
    (4, 256, 2, 8, 2100, 3),
    (2, 128, 2, 4, 1, None),
    (2, 128, 2, 4, 17, None),
    (2, 128, 3, 4, 300, None),
    (2, 128, 2, 8, 5000, None),
    (2, 128, 1, 4, 5000, 7),
]


@pytest.mark.parametrize("bits,head_dim,kv_heads,group,seq_len,n_splits", CASES)
@pytest.mark.parametrize("q_dtype", [torch.float32, torch.float16])
def test_matrix_kernel_matches_float32_products(hip_device, bits, head_dim, kv_heads, group, seq_len, n_splits,
                                                q_dtype):
    """Same inputs through both split kernels: equal to float32 rounding, and both at float32
    distance from the float64 decode of the same codes."""
    geo = dict(layers=1, kv_heads=kv_heads, group=group, head_dim=head_dim, seq_len=seq_len, bits=bits)
    c = _case(seq_len * 7 + head_dim + group + bits, capacity=seq_len + 5, q_dtype=q_dtype, q_scale=1.0,
              dev=hip_device, **geo)
    mx = _decode(c, capacity=seq_len + 5, f32_products=False, n_splits=n_splits, **geo)
    f32 = _decode(c, capacity=seq_len + 5, f32_products=True, n_splits=n_splits, **geo)
    ref = _float64_reference(c, **geo)
    scale = np.abs(ref).max()
    np.testing.assert_allclose(mx, f32, rtol=2e-5, atol=2e-6 * scale)
    err_mx = np.abs(mx - ref).max() / scale
    err_f32 = np.abs(f32 - ref).max() / scale
    assert err_mx < 2e-6, err_mx
    assert err_f32 < 2e-6, err_f32


@pytest.mark.parametrize("q_scale,bits", [(8.0, 4), (60.0, 4), (60.0, 2)])
def test_matrix_kernel_large_score_range(hip_device, q_scale, bits):
    """Scores spread over hundreds of log units (weights far below the maximum, running maxima
    that move mid-split).  A score of magnitude |s| carries ~|s| x (product precision) absolute
    error, which exp() turns into relative weight error: float32 products give 2^-24, the exact
    f16 splits (22 significant bits per factor) ~2^-21, so at q x 60 the matrix kernel sits at up
    to ~8x the float32 kernel's distance from the float64 decode (measured 8.2e-6 against
    2.1e-6), still far inside the 2e-3 bound."""
    geo = dict(layers=2, kv_heads=2, group=4, head_dim=128, seq_len=3000, bits=bits)
    c = _case(int(q_scale), capacity=3000, q_dtype=torch.float32, q_scale=q_scale, dev=hip_device, **geo)
    ref = _float64_reference(c, **geo)
    scale = np.abs(ref).max()
    for ns in (None, 1, 13):
        mx = _decode(c, capacity=3000, f32_products=False, n_splits=ns, **geo)
        f32 = _decode(c, capacity=3000, f32_products=True, n_splits=ns, **geo)
        err_mx = np.abs(mx - ref).max() / scale
        err_f32 = np.abs(f32 - ref).max() / scale
        assert err_mx <= 8 * err_f32 + 2e-6, (ns, err_mx, err_f32)
        assert err_mx < 2e-3  # the north-star bound (max-abs 2e-3 at unit-scale outputs)


@pytest.mark.parametrize("head_dim,bits", [(128, 4), (256, 4), (128, 2)])
def test_matrix_kernel_rotation_and_current_token(hip_device, head_dim, bits):
    """Query rotation, inverse output rotation and the current-token path agree with the float32
    kernel (both run the same epilogue arithmetic on different split products)."""
    geo = dict(layers=1, kv_heads=2, group=4, head_dim=head_dim, seq_len=700, bits=bits)
    c = _case(11, capacity=800, q_dtype=torch.float16, q_scale=1.0, dev=hip_device, **geo)
    gen = torch.Generator(device=hip_device).manual_seed(3)
    cur = (torch.randn((1, 2, head_dim), generator=gen, device=hip_device) * 0.5,
           torch.randn((1, 2, head_dim), generator=gen, device=hip_device) * 0.05)
    for ns in (None, 1, 5):
        for current in (None, cur):
            mx = _decode(c, capacity=800, f32_products=False, n_splits=ns, rotate=True, current=current, **geo)
            f32 = _decode(c, capacity=800, f32_products=True, n_splits=ns, rotate=True, current=current, **geo)
            np.testing.assert_allclose(mx, f32, rtol=2e-5, atol=2e-6 * np.abs(f32).max(), err_msg=f"{ns} {current is None}")


@pytest.mark.parametrize("head_dim,bits", [(128, 4), (256, 4), (128, 2)])
def test_matrix_kernel_empty_sequence(hip_device, head_dim, bits):
    """No rows, the matrix kernel forced: zeros without a current token (the reference's S = 0 case,
    cache_mlx.py:178-180), the current token's value alone with one (its softmax weight is 1) -- the
    same outputs as the float32 kernel, on one split and on several empty ones."""
    geo = dict(layers=1, kv_heads=2, group=4, head_dim=head_dim, seq_len=0, bits=bits)
    c = _case(17, capacity=8, q_dtype=torch.float32, q_scale=1.0, dev=hip_device, **geo)
    gen = torch.Generator(device=hip_device).manual_seed(4)
    cur = (torch.randn((1, 2, head_dim), generator=gen, device=hip_device),
           torch.randn((1, 2, head_dim), generator=gen, device=hip_device))
    for ns in (None, 1, 3):
        for current in (None, cur):
            mx = _decode(c, capacity=8, f32_products=False, n_splits=ns, rotate=True, current=current, **geo)
            f32 = _decode(c, capacity=8, f32_products=True, n_splits=ns, rotate=True, current=current, **geo)
            assert np.isfinite(mx).all(), (ns, current is None)
            if current is None:
                assert not mx.any() and not f32.any(), ns
            else:
                np.testing.assert_allclose(mx, f32, rtol=1e-6, atol=1e-6, err_msg=f"{ns}")
                # the current token's value (given in the rotated basis) rotated back, for every
                # query head of its KV head
                signs_l, signs_r = c["np"]["signs"]
                expect = o.rotation_inverse(np.repeat(current[1].cpu().numpy()[0], 4, axis=0), signs_l, signs_r)
                np.testing.assert_allclose(mx[0], expect, rtol=1e-5, atol=1e-5, err_msg=f"{ns}")


@pytest.mark.parametrize("bits,head_dim,group", [(4, 128, 4), (4, 64, 8), (2, 128, 4), (4, 256, 4)])
def test_matrix_kernel_repeatable_across_calls(hip_device, bits, head_dim, group):
    """The tiles are dealt statically, so repeated calls return identical bits (with and without a current
    token, one and several splits), and never pick up state an earlier call left; the result agrees with
    the float32-product kernel to float32 rounding."""
    geo = dict(layers=1, kv_heads=2, group=group, head_dim=head_dim, seq_len=9000)
    c = _case(6, capacity=9000, q_dtype=torch.float16, q_scale=3.0, dev=hip_device, bits=bits, **geo)
    gen = torch.Generator(device=hip_device).manual_seed(6)
    cur = (torch.randn((1, 2, head_dim), generator=gen, device=hip_device),
           torch.randn((1, 2, head_dim), generator=gen, device=hip_device))
    for current in (None, cur):
        for ns in (None, 3):
            kw = dict(capacity=9000, f32_products=False, n_splits=ns, rotate=True, current=current, bits=bits)
            first = _decode(c, **kw, **geo)
            for _ in range(4):
                np.testing.assert_array_equal(_decode(c, **kw, **geo), first)
            f32 = _decode(c, **{**kw, "f32_products": True}, **geo)
            np.testing.assert_allclose(f32, first, rtol=1e-5, atol=2e-6 * np.abs(first).max())
