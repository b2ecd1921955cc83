"""tq_decode_noalloc: the decode without a caller workspace, through the C ABI.

Its split-K partials live in the library's static per-GPU scratch array.  Two
calls in a row -- the second smaller than the first, so it runs over what the
first left in the scratch -- each give tq_decode's output on the same inputs:
the same kernels and split plan, so the outputs agree to float32 rounding (the
split kernel's wavefronts claim tiles dynamically, so the order in which a
workgroup adds its tiles, and with it the last bits, can differ between any two
calls).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _cache(dev, bits, head_dim, kv_heads, seq_len, seed):
    import torque_hip as th

    cfg = th.TorqueConfig(bit_width=bits, head_dim=head_dim, num_layers=1, kv_heads=kv_heads, rotation_seed=seed)
    cache = th.TorqueKVCacheHIP(config=cfg, initial_capacity=seq_len, decode_tail_capacity=0)
    gen = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn((1, kv_heads, seq_len, head_dim), generator=gen, device=dev)
    v = torch.randn((1, kv_heads, seq_len, head_dim), generator=gen, device=dev)
    cache.append_many(key=k, value=v)
    return cache


def _both(dev, cache, query, n_splits):
    """(tq_decode output, tq_decode_noalloc output) for one query [1, Hq, D]."""
    from torque_hip import _lib, ops
    from torque_hip._tensors import dtype_code

    st = cache._store
    cfg = cache.config
    hq = int(query.shape[1])
    flags = _lib.TQ_ROTATE_QUERY | _lib.TQ_INVERSE_OUTPUT
    stream = torch.cuda.current_stream(dev).cuda_stream
    common = (query.data_ptr(), dtype_code(query), 1, hq, cfg.kv_heads, cfg.head_dim, cfg.bit_width,
              st.key_codes.data_ptr(), st.value_codes.data_ptr(), st.capacity, st.length, st.key_centroids.data_ptr(),
              st.value_centroids.data_ptr(), st.signs_left.data_ptr(), st.signs_right.data_ptr(), flags, None, None,
              n_splits)
    ns = n_splits if n_splits > 0 else ops.plan_splits(1, cfg.kv_heads, hq, cfg.head_dim, st.length, dev,
                                                       bit_width=cfg.bit_width)
    ws = torch.empty(_lib.call("tq_decode_workspace_bytes", 1, cfg.kv_heads, hq, cfg.head_dim, ns, ops.num_cus(dev)),
                     dtype=torch.uint8, device=dev)
    ref = torch.empty((1, hq, cfg.head_dim), dtype=torch.float32, device=dev)
    got = torch.full_like(ref, float("nan"))
    _lib.call("tq_decode", *common, ws.data_ptr(), ws.numel(), ref.data_ptr(), stream)
    _lib.call("tq_decode_noalloc", *common, got.data_ptr(), stream)
    torch.cuda.synchronize(dev)
    return ref.cpu().numpy(), got.cpu().numpy()


def test_noalloc_matches_decode_on_two_calls(hip_device):
    big = _cache(hip_device, 4, 128, 4, 6000, seed=3)
    small = _cache(hip_device, 3, 64, 2, 900, seed=4)
    gen = torch.Generator(device=hip_device).manual_seed(5)
    q_big = torch.randn((1, 16, 128), generator=gen, device=hip_device).half()
    q_small = torch.randn((1, 4, 64), generator=gen, device=hip_device)
    for cache, q, ns in ((big, q_big, 0), (small, q_small, 0), (small, q_small, 3), (big, q_big, 1)):
        ref, got = _both(hip_device, cache, q, ns)
        assert np.isfinite(ref).all()
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_noalloc_rejects_oversized_plan(hip_device):
    from torque_hip import _lib

    # 4 layers x 64 query heads x 256 splits x D=256 partials: 64 MiB of scratch, beyond the 8 MiB array
    fake = 0x1000
    with pytest.raises(ValueError, match="bytes of scratch"):
        _lib.call("tq_decode_noalloc", fake, 0, 4, 64, 8, 256, 4, fake, fake, 1 << 20, 1 << 20, fake, fake, None, None,
                  0, None, None, 256, fake, None)
