"""Decode launches captured in a HIP graph and replayed.

The library allocates nothing inside a call and records no memset or copy,
only kernel launches, so its calls can be captured.  A ``tq_decode`` (split
kernel + merge kernel) and the allocation-free ``tq_decode_noalloc`` -- the
entry point meant for callers that capture -- are each captured once and
replayed several times, with the program's own eager decodes and
synchronisations between the replays.  Every replay must give the eager
result bit for bit: both split kernels deal their work statically and the
merge sums the splits in a fixed order.  The eager calls in between run other inputs and shapes, so a
replay that read state an earlier call left behind (workspace, scratch)
would show.
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


def _decode(cache, query, f32_products):
    from torque_hip.ops import packed_decode

    st, cfg = cache._store, cache.config
    return packed_decode(query, num_layers=1, query_heads=int(query.shape[1]), kv_heads=cfg.kv_heads,
                         head_dim=cfg.head_dim, bit_width=cfg.bit_width, key_codes=st.key_codes,
                         value_codes=st.value_codes, capacity=st.capacity, seq_len=st.length,
                         key_centroids=st.key_centroids, value_centroids=st.value_centroids,
                         signs_left=st.signs_left, signs_right=st.signs_right, rotate_query=True,
                         inverse_output=True, f32_products=f32_products, matrix_products=not f32_products)


def _noalloc(cache, query, out):
    from torque_hip import _lib
    from torque_hip._tensors import dtype_code

    st, cfg = cache._store, cache.config
    dev = query.device
    _lib.call("tq_decode_noalloc", query.data_ptr(), dtype_code(query), 1, int(query.shape[1]), cfg.kv_heads,
              cfg.head_dim, cfg.bit_width, st.key_codes.data_ptr(), st.value_codes.data_ptr(), st.capacity,
              st.length, st.key_centroids.data_ptr(), st.value_centroids.data_ptr(), st.signs_left.data_ptr(),
              st.signs_right.data_ptr(), _lib.TQ_ROTATE_QUERY | _lib.TQ_INVERSE_OUTPUT, None, None, 0,
              out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    return out


def _capture(dev, fn):
    """fn() captured once in a graph (after two warm-up calls on a side stream); returns (graph, output)."""
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


@pytest.mark.parametrize("f32_products", [True, False])
def test_captured_decode_replays(hip_device, f32_products):
    main = _cache(hip_device, 4, 128, 8, 16384, seed=21)
    other = _cache(hip_device, 4, 256, 2, 9000, seed=22)
    gen = torch.Generator(device=hip_device).manual_seed(23)
    q = torch.randn((1, 32, 128), generator=gen, device=hip_device).half()
    q_other = torch.randn((1, 8, 256), generator=gen, device=hip_device)
    ref = _decode(main, q, f32_products).cpu().numpy()
    graph, out = _capture(hip_device, lambda: _decode(main, q, f32_products))
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize(hip_device)
        np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"replay {rep}")
        _decode(other, q_other, f32_products)  # eager work on other buffers between the replays
        torch.cuda.synchronize(hip_device)


def test_captured_noalloc_replays(hip_device):
    """The no-allocation entry point in a graph: its split partials live in the library's static scratch,
    which the eager calls between replays (another shape and split plan) overwrite."""
    main = _cache(hip_device, 4, 128, 4, 6000, seed=31)
    other = _cache(hip_device, 3, 64, 2, 900, seed=32)
    gen = torch.Generator(device=hip_device).manual_seed(33)
    q = torch.randn((1, 16, 128), generator=gen, device=hip_device).half()
    q_other = torch.randn((1, 4, 64), generator=gen, device=hip_device)
    ref = _noalloc(main, q, torch.empty((1, 16, 128), dtype=torch.float32, device=hip_device)).clone()
    torch.cuda.synchronize(hip_device)
    ref = ref.cpu().numpy()
    out = torch.full((1, 16, 128), float("nan"), dtype=torch.float32, device=hip_device)
    out_other = torch.empty((1, 4, 64), dtype=torch.float32, device=hip_device)
    graph, _ = _capture(hip_device, lambda: _noalloc(main, q, out))
    for rep in range(4):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize(hip_device)
        got = out.cpu().numpy()
        assert np.isfinite(got).all(), rep
        np.testing.assert_array_equal(got, ref, err_msg=f"replay {rep}")
        _noalloc(other, q_other, out_other)
        torch.cuda.synchronize(hip_device)
