"""Concurrent decodes on two streams.

The kernels keep no state between calls and every call brings its own
workspace, so decodes issued on two streams at once return what they return
one after another, bit for bit (both split kernels deal their work
statically, so the summation order is fixed).  The reference runs on
one MLX stream (cache_mlx.py); the boundary here promises stateless,
stream-ordered launches, and this is that promise under overlap.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, seed, kv_heads, seq_len, head_dim=128, bits=4, group=4):
    rng = np.random.default_rng(seed)
    words = head_dim * bits // 32
    codes = lambda: torch.from_numpy(
        rng.integers(0, 2**32, size=(1, kv_heads, seq_len, words), dtype=np.uint64).astype(np.uint32).view(np.int32)
    ).to(dev)
    cent = lambda s: torch.from_numpy((np.sort(rng.normal(size=1 << bits)) * s).astype(np.float32)).to(dev)
    q = torch.from_numpy(rng.normal(size=(1, kv_heads * group, head_dim)).astype(np.float32)).to(dev, torch.float16)
    return dict(query=q, key_codes=codes(), value_codes=codes(), key_centroids=cent(1.5), value_centroids=cent(0.1),
                num_layers=1, query_heads=kv_heads * group, kv_heads=kv_heads, head_dim=head_dim, bit_width=bits,
                capacity=seq_len, seq_len=seq_len)


@pytest.mark.parametrize("f32_products", [True, False])
def test_two_streams_match_sequential(hip_device, f32_products):
    from torque_hip.ops import packed_decode

    cases = [_inputs(hip_device, 1, kv_heads=8, seq_len=16384), _inputs(hip_device, 2, kv_heads=4, seq_len=20000)]
    decode = lambda c: packed_decode(**c, f32_products=f32_products, matrix_products=not f32_products)
    ref = [decode(c).cpu().numpy() for c in cases]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(hip_device), torch.cuda.Stream(hip_device)
    for rep in range(3):
        with torch.cuda.stream(s1):
            a = decode(cases[0])
        with torch.cuda.stream(s2):
            b = decode(cases[1])
        torch.cuda.synchronize()
        for got, exp in zip((a.cpu().numpy(), b.cpu().numpy()), ref):
            np.testing.assert_array_equal(got, exp, err_msg=f"rep {rep}")


def test_step_timed_binds_caller_events(hip_device):
    """tq_decode_step_timed: the same output as tq_decode, with the caller's events bound to the split and
    the merge launches (both elapsed times positive); one merge event alone is refused."""
    import ctypes

    from torque_hip import _lib, ops
    from torque_hip._tensors import dtype_code

    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    evs = [ctypes.c_void_p() for _ in range(4)]
    for e in evs:
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
    c = _inputs(hip_device, 3, kv_heads=8, seq_len=16384)
    flags = 0
    ns = ops.plan_splits(1, 8, 32, 128, 16384, hip_device, bit_width=4, flags=flags)
    assert ns > 1
    ws = ops.workspace_for(1, 8, 32, 128, ns, hip_device)
    ref = ops.packed_decode(**c, n_splits=ns)
    out = torch.full_like(ref, float("nan"))
    stream = torch.cuda.current_stream(hip_device).cuda_stream
    args = (c["query"].data_ptr(), dtype_code(c["query"]), 1, 32, 8, 128, 4, c["key_codes"].data_ptr(),
            c["value_codes"].data_ptr(), 16384, 16384, c["key_centroids"].data_ptr(), c["value_centroids"].data_ptr(),
            None, None, flags, None, None, ns, ws.data_ptr(), ws.numel(), out.data_ptr(), stream)
    _lib.call("tq_decode_step_timed", *args, *evs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), ref.cpu().numpy())
    for a, b in ((evs[0], evs[1]), (evs[2], evs[3])):
        hip.hipEventSynchronize(b)
        ms = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        assert 0.0 < ms.value < 50.0
    with pytest.raises(ValueError, match="both be given"):
        _lib.call("tq_decode_step_timed", *args, evs[0], evs[1], evs[2], None)
    torch.cuda.synchronize()
    for e in evs:
        hip.hipEventDestroy(e)
