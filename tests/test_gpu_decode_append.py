"""tq_decode_append: one launch that packs the new token and decodes with it.

Checked against the two-launch sequence it replaces (append, then decode over
the grown cache): the packed words must be identical and the outputs equal to
float rounding; and against the oracle's append-then-decode.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torque_oracle as o

pytestmark = pytest.mark.gpu


def _pair(bits, head_dim, layers, kv_heads, capacity, fused=False, strategy="split_batched"):
    import torque_hip as th

    cfg = th.TorqueConfig(bit_width=bits, head_dim=head_dim, num_layers=layers, kv_heads=kv_heads, fused_weights=fused)
    kw = dict(config=cfg, initial_capacity=capacity, decode_tail_capacity=0, decode_strategy=strategy)
    return th.TorqueKVCacheHIP(**kw), th.TorqueKVCacheHIP(**kw)


def _codes(cache):
    s = cache.sequence_length
    return tuple(t[:, :, :s].cpu().numpy() for t in (cache._key_codes, cache._value_codes))


@pytest.mark.parametrize(
    "bits,head_dim,layers,kv_heads,group,prefill",
    [
        (4, 128, 1, 2, 4, 0),
        (4, 128, 2, 2, 4, 37),
        (3, 64, 1, 4, 4, 300),
        (2, 256, 1, 2, 2, 513),
        (4, 256, 1, 1, 1, 5),
        (4, 256, 1, 2, 4, 300),
        (4, 64, 1, 2, 8, 2100),
        (3, 128, 1, 3, 3, 1000),
    ],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_decode_append_matches_append_then_decode(hip_device, bits, head_dim, layers, kv_heads, group, prefill, dtype):
    gen = torch.Generator(device=hip_device).manual_seed(bits * 1000 + head_dim + prefill)
    a, b = _pair(bits, head_dim, layers, kv_heads, capacity=64)
    hq = kv_heads * group
    if prefill:
        k = torch.randn((layers, kv_heads, prefill, head_dim), generator=gen, device=hip_device).to(dtype)
        v = torch.randn((layers, kv_heads, prefill, head_dim), generator=gen, device=hip_device).to(dtype)
        a.append_many(key=k, value=v)
        b.append_many(key=k, value=v)
    for step in range(3):
        q = torch.randn((layers, hq, head_dim), generator=gen, device=hip_device).to(dtype)
        k = torch.randn((layers, kv_heads, head_dim), generator=gen, device=hip_device).to(dtype)
        v = torch.randn((layers, kv_heads, head_dim), generator=gen, device=hip_device).to(dtype)
        got = a.decode_append(query=q, key=k, value=v, return_numpy=False).cpu().numpy()
        b.append(key=k, value=v)
        exp = b.decode(query=q, return_numpy=False).cpu().numpy()
        assert a.sequence_length == b.sequence_length == prefill + step + 1
        for x, y in zip(_codes(a), _codes(b)):
            np.testing.assert_array_equal(x, y)
        np.testing.assert_allclose(got, exp, atol=2e-6, rtol=1e-5, err_msg=f"step {step}")


@pytest.mark.parametrize("q_dtype,kv_dtype", [(torch.float16, torch.float32), (torch.float32, torch.float16)])
def test_decode_append_mixed_dtypes(hip_device, q_dtype, kv_dtype):
    """The new token is quantized from its own values whatever the query's dtype (the reference quantizes
    float32 K/V, cache_mlx.py:442-466): codes equal append()'s and the oracle's on float32 K/V, so an fp16
    query never rounds fp32 keys before they are packed."""
    gen = torch.Generator(device=hip_device).manual_seed(77)
    a, b = _pair(4, 128, 1, 2, capacity=64)
    model = o.OracleCache(bit_width=4, head_dim=128, num_layers=1, kv_heads=2,
                          key_centroids=a.key_codebook.centroids, value_centroids=a.value_codebook.centroids,
                          signs_left=a.rotation.signs_left, signs_right=a.rotation.signs_right)
    for step in range(4):
        q = torch.randn((1, 8, 128), generator=gen, device=hip_device).to(q_dtype)
        k = (torch.randn((1, 2, 128), generator=gen, device=hip_device) * 3).to(kv_dtype)
        v = (torch.randn((1, 2, 128), generator=gen, device=hip_device) * 3).to(kv_dtype)
        got = a.decode_append(query=q, key=k, value=v, return_numpy=False).cpu().numpy()
        b.append(key=k, value=v)
        exp = b.decode(query=q, return_numpy=False).cpu().numpy()
        model.append(k.float().cpu().numpy()[:, :, None], v.float().cpu().numpy()[:, :, None])
        for x, y, m in zip(_codes(a), _codes(b), (model.k_codes, model.v_codes)):
            np.testing.assert_array_equal(x, y)
            np.testing.assert_array_equal(x.view(np.uint32), m)
        np.testing.assert_allclose(got, exp, atol=2e-6, rtol=1e-5, err_msg=f"step {step}")
        oracle_out = model.decode(q.float().cpu().numpy())[0]
        np.testing.assert_allclose(got.reshape(oracle_out.shape), oracle_out, atol=2e-5, rtol=1e-4,
                                   err_msg=f"step {step}")


def test_mixed_kv_dtypes_quantize_at_float32(hip_device):
    """append() and decode-with-current with an fp16 key and an fp32 value (or the reverse) quantize both at
    float32: the codes equal those of the same token given as two float32 tensors."""
    gen = torch.Generator(device=hip_device).manual_seed(78)
    for kd, vd in ((torch.float16, torch.float32), (torch.float32, torch.float16)):
        a, b = _pair(3, 64, 1, 2, capacity=16)
        for _ in range(3):
            k = (torch.randn((1, 2, 64), generator=gen, device=hip_device) * 2).to(kd)
            v = (torch.randn((1, 2, 64), generator=gen, device=hip_device) * 2).to(vd)
            a.append(key=k, value=v)
            b.append(key=k.float(), value=v.float())
        for x, y in zip(_codes(a), _codes(b)):
            np.testing.assert_array_equal(x, y)
        q = torch.randn((1, 8, 64), generator=gen, device=hip_device)
        np.testing.assert_allclose(a.decode(query=q, return_numpy=False).cpu().numpy(),
                                   b.decode(query=q, return_numpy=False).cpu().numpy(), atol=1e-6)


@pytest.mark.parametrize("bits,head_dim", [(4, 128), (4, 256), (2, 128)])
def test_decode_append_against_oracle_and_split_counts(hip_device, bits, head_dim):
    """3000 rows: 1 and 3 splits run the matrix kernel (24 and 8 blocks of 128 rows per split), 64 splits the
    float32 kernel; 5 and 7 splits force the matrix kernel onto uneven shares of the 24 blocks.  The appending
    split 0 takes the lightest share at 3 and 5 splits (splits 1.. alone would need 12 and 6 blocks each) and
    no rows at 7 and 64 (the other splits take 4 blocks each of 128 rows, or 2-3 of the float32 kernel's,
    as a deal over all the splits would).  Every output matches the oracle's append-then-decode."""
    import torque_hip as th
    from torque_hip import _lib
    from torque_hip.ops import packed_decode_append

    D = head_dim

    rng = np.random.default_rng(5)
    cfg = th.TorqueConfig(bit_width=bits, head_dim=D, num_layers=1, kv_heads=2)
    cache = th.TorqueKVCacheHIP(config=cfg, initial_capacity=4096, decode_tail_capacity=0)
    k0 = rng.normal(size=(1, 2, 3000, D)).astype(np.float32)
    v0 = rng.normal(size=(1, 2, 3000, D)).astype(np.float32)
    cache.append_many(key=k0, value=v0)
    q = rng.normal(size=(8, D)).astype(np.float32)
    kn = rng.normal(size=(2, D)).astype(np.float32)
    vn = rng.normal(size=(2, D)).astype(np.float32)
    st = cache._store
    kernels = [_lib.split_kernel(2, 8, D, bits, 3, _lib.TQ_F32, 3000, n_splits=ns) for ns in (1, 3, 64)]
    mx_name = f"decode_mx_kernel<{D},false>" if bits == 4 else f"decode_mx_kernel<{D},false,{bits}>"
    assert kernels[:2] == [mx_name] * 2 and kernels[2].startswith("decode_kernel<"), kernels
    forced = (5, 7)
    for ns in forced:
        assert _lib.split_kernel(2, 8, D, bits, 3 | _lib.TQ_MATRIX_PRODUCTS, _lib.TQ_F32, 3000, n_splits=ns) == mx_name
    qd = torch.from_numpy(q).to(hip_device).reshape(1, 8, D)
    knd = torch.from_numpy(kn).to(hip_device).reshape(1, 2, 1, D)
    vnd = torch.from_numpy(vn).to(hip_device).reshape(1, 2, 1, D)
    split_counts = (1, 3, 64) + forced
    outs = []
    for ns in split_counts:
        st.length = 3000  # rewrite the same token at the same row each time
        if ns in forced:
            got = packed_decode_append(
                qd, knd, vnd, num_layers=1, query_heads=8, kv_heads=2, head_dim=D, bit_width=bits,
                key_codes=st.key_codes, value_codes=st.value_codes, capacity=st.capacity, seq_len=3000,
                key_centroids=st.key_centroids, value_centroids=st.value_centroids,
                key_boundaries=st.key_boundaries, value_boundaries=st.value_boundaries,
                signs_left=st.signs_left, signs_right=st.signs_right, rotate_query=True, inverse_output=True,
                n_splits=ns, matrix_products=True)
            st.length = 3001
        else:
            got = st.decode_append(qd, knd, vnd, rotate_query=True, inverse_output=True, rotate_keys=True,
                                   rotate_values=True, n_splits=ns)
        outs.append(got.cpu().numpy()[0])
    model = o.OracleCache(bit_width=bits, head_dim=D, num_layers=1, kv_heads=2,
                          key_centroids=cache.key_codebook.centroids, value_centroids=cache.value_codebook.centroids,
                          signs_left=cache.rotation.signs_left, signs_right=cache.rotation.signs_right)
    model.append(np.concatenate([k0, kn.reshape(1, 2, 1, D)], axis=2), np.concatenate([v0, vn.reshape(1, 2, 1, D)], axis=2))
    exp = model.decode(q.reshape(1, 8, D))[0]
    cache.sequence_length = 3001
    kc, vc = _codes(cache)
    np.testing.assert_array_equal(kc.view(np.uint32), model.k_codes)
    np.testing.assert_array_equal(vc.view(np.uint32), model.v_codes)
    for ns, out in zip(split_counts, outs):
        np.testing.assert_allclose(out, exp, atol=2e-6, rtol=1e-5, err_msg=f"n_splits {ns}")


def test_decode_append_flags_growth_and_errors(hip_device):
    from torque_hip import _lib

    rng = np.random.default_rng(9)
    for fused in (False, True):
        a, b = _pair(3, 64, 1, 2, capacity=2, fused=fused, strategy="fused_per_head")
        a.rotate_values_on_append = b.rotate_values_on_append = False
        for step in range(5):  # grows 2 -> 4 -> 8
            q = rng.normal(size=(4, 64)).astype(np.float32)
            k = rng.normal(size=(2, 64)).astype(np.float32)
            v = rng.normal(size=(2, 64)).astype(np.float32)
            got = a.decode_append(query=q, key=k, value=v)
            b.append(key=k, value=v)
            np.testing.assert_allclose(got, b.decode(query=q), atol=2e-6, rtol=1e-5)
        assert a.capacity == b.capacity == 8
        for x, y in zip(_codes(a), _codes(b)):
            np.testing.assert_array_equal(x, y)
    with pytest.raises(ValueError, match="single token"):
        a.decode_append(query=np.zeros((4, 64), np.float32), key=np.zeros((2, 3, 64), np.float32),
                        value=np.zeros((2, 3, 64), np.float32))
    st = a._store
    q = torch.zeros((1, 4, 64), device=hip_device)
    kv = torch.zeros((1, 2, 1, 64), device=hip_device)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=hip_device)
    out = torch.empty((1, 4, 64), device=hip_device)
    with pytest.raises(ValueError, match="slab is full"):
        _lib.call("tq_decode_append", q.data_ptr(), _lib.TQ_F32, kv.data_ptr(), kv.data_ptr(), _lib.TQ_F32, 1, 4, 2,
                  64, 3, st.key_codes.data_ptr(), st.value_codes.data_ptr(), st.capacity, st.capacity,
                  st.key_centroids.data_ptr(), st.value_centroids.data_ptr(), st.key_boundaries.data_ptr(),
                  st.value_boundaries.data_ptr(), st.signs_left.data_ptr(), st.signs_right.data_ptr(), 3, 3, 0,
                  ws.data_ptr(), ws.numel(), out.data_ptr(), None)
