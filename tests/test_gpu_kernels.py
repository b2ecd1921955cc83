"""GPU parity of the HIP kernels against the CPU oracle, op by op.

Mirrors the reference's device tests (tests/test_mlx_ops.py, test_rotation.py:28-50,
test_quantization.py:77-111).  Integer outputs (packed words) must be
bit-identical; the rotation is bit-identical too (same float32 butterflies);
decode outputs are compared within float32 accumulation-order tolerance.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torque_oracle as o

pytestmark = pytest.mark.gpu

BITS = [2, 3, 4]
DIMS = [64, 128, 256]


def _u32(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("head_dim", DIMS)
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_rotation_bit_exact(hip_device, head_dim, dtype):
    # test_rotation.py:28-50 (the reference allows 1e-5; the FWHT here is bit-identical)
    import torque_hip as th

    rng = np.random.default_rng(7)
    x = rng.normal(size=(37, head_dim)).astype(dtype)
    spec = th.RotationSpec.from_seed(head_dim, 13)
    got = spec.apply(x)
    exp = o.rotation_apply(x.astype(np.float32), spec.signs_left, spec.signs_right)
    np.testing.assert_array_equal(got, exp)
    back = spec.inverse(got)
    np.testing.assert_array_equal(back, o.rotation_inverse(exp, spec.signs_left, spec.signs_right))
    np.testing.assert_allclose(back, x.astype(np.float32), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("head_dim", DIMS)
def test_quantize_and_pack_rows_bit_exact(hip_device, bits, head_dim):
    # test_mlx_ops.py:65-86
    import torque_hip as th

    cb = th.build_uniform_codebook(bits)
    rng = np.random.default_rng(12)
    values = rng.uniform(-1.0, 1.0, size=(5, head_dim)).astype(np.float32)
    got = th.quantize_and_pack_rows(values, th.codebook_boundaries(cb), bit_width=bits, head_dim=head_dim)
    np.testing.assert_array_equal(_u32(got), o.pack_indices_batched(o.quantize_argmin(values, cb.centroids), bits))
    # Larger, Gaussian codebook, values spanning all codes and beyond.
    gcb = th.build_gaussian_codebook(bits, seed=bits)
    big = rng.normal(0.0, 1.7, size=(1000, head_dim)).astype(np.float32)
    got = th.quantize_and_pack_rows(big, th.codebook_boundaries(gcb), bit_width=bits, head_dim=head_dim)
    exp = o.pack_indices_batched(o.quantize_boundary_count(big, o.codebook_boundaries(gcb.centroids)), bits)
    np.testing.assert_array_equal(_u32(got), exp)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("head_dim", DIMS)
def test_quantize_and_pack_rows_dual_bit_exact(hip_device, bits, head_dim):
    # test_mlx_ops.py:89-120
    import torque_hip as th

    a_cb = th.Codebook(bit_width=bits, centroids=np.linspace(-1.0, 1.0, 1 << bits, dtype=np.float32))
    b_cb = th.Codebook(bit_width=bits, centroids=np.linspace(-0.75, 0.75, 1 << bits, dtype=np.float32))
    rng = np.random.default_rng(13)
    va = rng.uniform(-1.0, 1.0, size=(5, head_dim)).astype(np.float32)
    vb = rng.uniform(-0.75, 0.75, size=(5, head_dim)).astype(np.float32)
    ga, gb = th.quantize_and_pack_rows_dual(
        va, vb, th.codebook_boundaries(a_cb), th.codebook_boundaries(b_cb), bit_width=bits, head_dim=head_dim
    )
    np.testing.assert_array_equal(_u32(ga), o.pack_indices_batched(o.quantize_argmin(va, a_cb.centroids), bits))
    np.testing.assert_array_equal(_u32(gb), o.pack_indices_batched(o.quantize_argmin(vb, b_cb.centroids), bits))


def test_quantize_tie_break_on_device(hip_device):
    # test_quantization.py:89-98: exact midpoints go to the lower code
    import torque_hip as th

    cb = th.Codebook(bit_width=2, centroids=np.array([-1.0, -0.25, 0.25, 1.0], dtype=np.float32))
    row = np.zeros((1, 64), dtype=np.float32)
    row[0, :3] = [-0.625, 0.0, 0.625]
    row[0, 3:6] = [-0.9, -0.2, 0.3]
    got = _u32(th.quantize_and_pack_rows(row, th.codebook_boundaries(cb), bit_width=2, head_dim=64))
    codes = o.unpack_indices(got[0], 2, 64)
    np.testing.assert_array_equal(codes[:6], [0, 1, 2, 0, 1, 2])


def test_quantize_and_pack_rejects_bad_shapes(hip_device):
    import torque_hip as th

    with pytest.raises(ValueError, match="values must have shape"):
        th.quantize_and_pack_rows(np.zeros((3, 60), np.float32), np.zeros(15, np.float32), bit_width=4, head_dim=64)
    with pytest.raises(ValueError, match="boundaries must have shape"):
        th.quantize_and_pack_rows(np.zeros((3, 64), np.float32), np.zeros(7, np.float32), bit_width=4, head_dim=64)


def _packed_case(bits, head_dim, batch, seq_len, seed):
    cb = o.uniform_codebook(bits)
    rng = np.random.default_rng(seed)
    q = rng.uniform(-1.0, 1.0, size=(batch, head_dim)).astype(np.float32)
    k = rng.uniform(-1.0, 1.0, size=(batch, seq_len, head_dim)).astype(np.float32)
    v = rng.uniform(-1.0, 1.0, size=(batch, seq_len, head_dim)).astype(np.float32)
    ki, vi = o.quantize_argmin(k, cb), o.quantize_argmin(v, cb)
    return cb, q, ki, vi, o.pack_indices_batched(ki, bits), o.pack_indices_batched(vi, bits), rng


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("head_dim", DIMS)
def test_decode_packed_attention_single_head(hip_device, bits, head_dim):
    # test_mlx_ops.py:19-62 (S=7, atol 1e-5)
    import torque_hip as th

    cb, q, ki, vi, kp, vp, _ = _packed_case(bits, head_dim, 1, 7, 0)
    got = th.decode_packed_attention(q[0], kp[0], vp[0], cb, cb, bit_width=bits, head_dim=head_dim)
    exp = o.streaming_attention_decode(q[0], cb[ki[0]], cb[vi[0]])
    np.testing.assert_allclose(got.cpu().numpy(), exp, atol=1e-5, rtol=1e-5)


def test_fused_and_split_decode_match(hip_device):
    # test_mlx_ops.py:123-168
    import torque_hip as th

    cb, q, ki, vi, kp, vp, _ = _packed_case(4, 64, 1, 11, 1)
    fused = th.decode_packed_attention(q[0], kp[0], vp[0], cb, cb, bit_width=4, head_dim=64)
    split = th.decode_packed_attention_split(q[0], kp[0], vp[0], cb, cb, bit_width=4, head_dim=64)
    np.testing.assert_allclose(fused.cpu().numpy(), split.cpu().numpy(), atol=1e-5, rtol=1e-5)
    exp = o.streaming_attention_decode(q[0], cb[ki[0]], cb[vi[0]])
    np.testing.assert_allclose(split.cpu().numpy(), exp, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("head_dim", DIMS)
def test_split_batched_matches_reference(hip_device, bits, head_dim):
    # test_mlx_ops.py:171-221 (B=5, S=9)
    import torque_hip as th

    cb, q, ki, vi, kp, vp, _ = _packed_case(bits, head_dim, 5, 9, 2)
    got = th.decode_packed_attention_split_batched(q, kp, vp, cb, cb, bit_width=bits, head_dim=head_dim)
    exp = np.stack([o.streaming_attention_decode(q[b], cb[ki[b]], cb[vi[b]]) for b in range(5)])
    np.testing.assert_allclose(got.cpu().numpy(), exp, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("head_dim", DIMS)
@pytest.mark.parametrize("seq_len", [0, 9])
def test_split_batched_with_current_matches_reference(hip_device, head_dim, seq_len):
    # test_mlx_ops.py:224-284; seq_len 0 returns the current values (mlx_ops.py:631-632)
    import torque_hip as th

    cb, q, ki, vi, kp, vp, rng = _packed_case(4, head_dim, 5, seq_len, 21)
    ck = rng.uniform(-1.0, 1.0, size=(5, head_dim)).astype(np.float32)
    cv = rng.uniform(-1.0, 1.0, size=(5, head_dim)).astype(np.float32)
    got = th.decode_packed_attention_split_batched_with_current(q, kp, vp, cb, cb, ck, cv, bit_width=4, head_dim=head_dim)
    exp = np.stack(
        [
            o.streaming_attention_decode(
                q[b], np.concatenate([cb[ki[b]], ck[b : b + 1]]), np.concatenate([cb[vi[b]], cv[b : b + 1]])
            )
            for b in range(5)
        ]
    )
    np.testing.assert_allclose(got.cpu().numpy(), exp, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("bits", BITS)
def test_staged_ops_match_reference(hip_device, bits):
    """score_packed_query_batched / softmax / accumulate_packed_values_batched (mlx_ops.py:501-568)."""
    from torque_hip import ops

    cb, q, ki, vi, kp, vp, _ = _packed_case(bits, 128, 3, 300, 5)
    scores = ops.score_packed_query_batched(q, kp, cb, bit_width=bits, head_dim=128).cpu().numpy()
    np.testing.assert_allclose(scores, np.einsum("bd,bsd->bs", q, cb[ki]), atol=1e-4, rtol=1e-5)
    w = ops.softmax_rows(scores, 1.0 / np.sqrt(128)).cpu().numpy()
    s = scores / np.sqrt(128)
    ew = np.exp(s - s.max(axis=1, keepdims=True))
    np.testing.assert_allclose(w, ew / ew.sum(axis=1, keepdims=True), rtol=1e-5, atol=1e-7)
    out = ops.accumulate_packed_values_batched(w, vp, cb, bit_width=bits, head_dim=128).cpu().numpy()
    np.testing.assert_allclose(out, np.einsum("bs,bsd->bd", w, cb[vi]), atol=1e-5, rtol=1e-5)
    # the lane groups' partial sums are added in a fixed order: repeated calls agree bit for bit
    for _ in range(3):
        again = ops.accumulate_packed_values_batched(w, vp, cb, bit_width=bits, head_dim=128).cpu().numpy()
        np.testing.assert_array_equal(again, out)


@pytest.mark.parametrize("head_dim", DIMS)
@pytest.mark.parametrize("kv_dtype", [np.float16, np.float32])
def test_dense_decode_matches_textbook(hip_device, head_dim, kv_dtype):
    """The fp16-dense comparator kernel (and its fp32 form) against float64 attention."""
    from torque_hip import ops

    rng = np.random.default_rng(head_dim)
    L, hkv, hq, s, cap = 2, 2, 8, 1000, 1024
    q = rng.normal(size=(L, hq, head_dim)).astype(np.float32)
    k = rng.normal(size=(L, hkv, cap, head_dim)).astype(kv_dtype)
    v = rng.normal(size=(L, hkv, cap, head_dim)).astype(kv_dtype)
    dev = hip_device
    got = ops.dense_decode(
        torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
        num_layers=L, query_heads=hq, kv_heads=hkv, head_dim=head_dim, capacity=cap, seq_len=s,
    ).cpu().numpy()
    idx = np.arange(hq) // (hq // hkv)
    exp = o.attention_decode_dense(q, k[:, idx, :s].astype(np.float32), v[:, idx, :s].astype(np.float32))
    np.testing.assert_allclose(got, exp, atol=2e-5, rtol=1e-4)
