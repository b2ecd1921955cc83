"""decode_kernel's wide instance: 3 tokens per lane group, 48-row workgroup iterations.

It exists for 4-bit rows at head_dim 256 in groups of 4 query heads, and the
host runs it where the 32-row deal would end on a nearly empty iteration:
8193..9216 rows over 64 splits (a 24-layer decode loop at 8K tokens).  At
8200 rows x 4 KV / 16 query heads the tests check, on that instance:
- decode against the oracle's decode of the same cache;
- decode_append against append-then-decode (identical codes) and the oracle;
- the per-vector-scale kernel against the same call at 128 splits, which runs
  the 2-token instance (to float32 rounding: the summation order differs).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torque_oracle as o

pytestmark = pytest.mark.gpu

L, HKV, HQ, D, BITS, ROWS = 1, 4, 16, 256, 4, 8200
WIDE = "decode_kernel<PackedB4,256,4,3>"


def _wide(rows, flags=0, dtype=None, n_splits=0):
    from torque_hip import _lib

    return _lib.split_kernel(HKV, HQ, D, BITS, flags, _lib.TQ_F16 if dtype is None else dtype, rows, n_splits=n_splits)


def _cache(rng, rows):
    import torque_hip as th

    cfg = th.TorqueConfig(bit_width=BITS, head_dim=D, num_layers=L, kv_heads=HKV, rotation_seed=9)
    cache = th.TorqueKVCacheHIP(config=cfg, initial_capacity=rows + 8, decode_tail_capacity=0)
    k = rng.normal(size=(L, HKV, rows, D)).astype(np.float32)
    v = rng.normal(size=(L, HKV, rows, D)).astype(np.float32)
    cache.append_many(key=k, value=v)
    model = o.OracleCache(bit_width=BITS, head_dim=D, num_layers=L, kv_heads=HKV,
                          key_centroids=cache.key_codebook.centroids, value_centroids=cache.value_codebook.centroids,
                          signs_left=cache.rotation.signs_left, signs_right=cache.rotation.signs_right)
    model.append(k, v)
    return cache, model


@pytest.mark.parametrize("q_dtype", [torch.float32, torch.float16])
def test_wide_decode_matches_oracle(hip_device, q_dtype):
    from torque_hip import _lib

    assert _wide(ROWS, dtype=_lib.TQ_F16 if q_dtype == torch.float16 else _lib.TQ_F32) == WIDE
    assert _wide(8192) != WIDE  # the narrow instance at 8192 rows (4 against 3 iterations)
    rng = np.random.default_rng(41)
    cache, model = _cache(rng, ROWS)
    q = rng.normal(size=(L, HQ, D)).astype(np.float32)
    got = cache.decode(query=torch.from_numpy(q).to(hip_device, q_dtype), return_numpy=False).cpu().numpy()
    exp = model.decode(q if q_dtype == torch.float32 else q.astype(np.float16).astype(np.float32))
    np.testing.assert_allclose(got.reshape(exp.shape), exp, atol=2e-5, rtol=1e-4)


def test_wide_decode_append_matches_append_then_decode(hip_device):
    rng = np.random.default_rng(42)
    a, model = _cache(rng, 8192)
    b, _ = _cache(np.random.default_rng(42), 8192)
    for step in range(3):
        assert _wide(8192 + step + 1) == WIDE
        q = rng.normal(size=(L, HQ, D)).astype(np.float32)
        kn = rng.normal(size=(L, HKV, D)).astype(np.float32)
        vn = rng.normal(size=(L, HKV, D)).astype(np.float32)
        td = lambda x: torch.from_numpy(x).to(hip_device)  # noqa: E731
        got = a.decode_append(query=td(q), key=td(kn), value=td(vn), return_numpy=False).cpu().numpy()
        b.append(key=td(kn), value=td(vn))
        exp = b.decode(query=td(q), return_numpy=False).cpu().numpy()
        s = a.sequence_length
        assert s == b.sequence_length == 8192 + step + 1
        for x, y in ((a._key_codes, b._key_codes), (a._value_codes, b._value_codes)):
            np.testing.assert_array_equal(x[:, :, :s].cpu().numpy(), y[:, :, :s].cpu().numpy())
        np.testing.assert_allclose(got, exp, atol=2e-6, rtol=1e-5, err_msg=f"step {step}")
        model.append(kn[:, :, None], vn[:, :, None])
        oracle_out = model.decode(q)
        np.testing.assert_allclose(got.reshape(oracle_out.shape), oracle_out, atol=2e-5, rtol=1e-4,
                                   err_msg=f"step {step}")


def test_wide_scaled_decode_matches_narrow(hip_device):
    from torque_hip import _lib
    from torque_hip.ops import packed_decode

    assert _wide(ROWS, flags=_lib.TQ_F32_PRODUCTS) == WIDE
    assert _wide(ROWS, flags=_lib.TQ_F32_PRODUCTS, n_splits=128) == "decode_kernel<PackedB4,256,4>"
    rng = np.random.default_rng(43)
    words = D * BITS // 32
    dev = hip_device
    codes = lambda: torch.from_numpy(  # noqa: E731
        rng.integers(0, 2**32, size=(L, HKV, ROWS, words), dtype=np.uint64).astype(np.uint32).view(np.int32)).to(dev)
    scales = lambda: torch.from_numpy(rng.lognormal(0.0, 1.0, size=(L, HKV, ROWS)).astype(np.float32)).to(dev)  # noqa: E731
    cent = lambda s: torch.from_numpy((np.sort(rng.normal(size=16)) * s).astype(np.float32)).to(dev)  # noqa: E731
    args = dict(num_layers=L, query_heads=HQ, kv_heads=HKV, head_dim=D, bit_width=BITS, key_codes=codes(),
                value_codes=codes(), capacity=ROWS, seq_len=ROWS, key_centroids=cent(0.3), value_centroids=cent(0.5),
                key_scales=scales(), value_scales=scales())
    q = torch.from_numpy(rng.normal(size=(L, HQ, D)).astype(np.float32)).to(dev, torch.float16)
    wide = packed_decode(q, **args).cpu().numpy()
    narrow = packed_decode(q, **args, n_splits=128).cpu().numpy()
    assert np.isfinite(wide).all()
    np.testing.assert_allclose(wide, narrow, rtol=1e-5, atol=1e-6 * np.abs(narrow).max())
