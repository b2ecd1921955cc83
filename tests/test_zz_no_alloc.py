"""tq_decode_noalloc: the decode without a caller workspace, through the C ABI.

Its split-K partials live in the library's static per-GPU scratch array.  Two
calls in a row -- the second smaller than the first, so it runs over what the
first left in the scratch -- each give tq_decode's output on the same inputs,
bit for bit: the same kernels, split plan and summation order.
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
        np.testing.assert_array_equal(got, ref)


def test_noalloc_rejects_oversized_plan(hip_device):
    from torque_hip import _lib

    # 4 layers x 64 query heads x 256 splits x D=256 partials: 64 MiB of scratch, beyond the 8 MiB array
    fake = 0x1000
    with pytest.raises(ValueError, match="bytes of scratch"):
        _lib.call("tq_decode_noalloc", fake, 0, 4, 64, 8, 256, 4, fake, fake, 1 << 20, 1 << 20, fake, fake, None, None,
                  0, None, None, 256, fake, None)


def test_noalloc_matrix_kernel_matches_decode_bit_for_bit(hip_device):
    """The matrix split kernel forced on two shapes, two calls in a row (the second smaller): both entry points
    sum the same tiles in the same order, identical bits."""
    from torque_hip import _lib
    from torque_hip._tensors import dtype_code

    big = _cache(hip_device, 4, 128, 4, 6000, seed=13)
    small = _cache(hip_device, 2, 128, 2, 1500, seed=14)
    gen = torch.Generator(device=hip_device).manual_seed(15)
    stream = torch.cuda.current_stream(hip_device).cuda_stream
    flags = _lib.TQ_ROTATE_QUERY | _lib.TQ_INVERSE_OUTPUT | _lib.TQ_MATRIX_PRODUCTS
    for cache, hq, ns in ((big, 16, 6), (small, 8, 3)):
        st, cfg = cache._store, cache.config
        q = torch.randn((1, hq, cfg.head_dim), generator=gen, device=hip_device).half()
        common = (q.data_ptr(), dtype_code(q), 1, hq, cfg.kv_heads, cfg.head_dim, cfg.bit_width,
                  st.key_codes.data_ptr(), st.value_codes.data_ptr(), st.capacity, st.length,
                  st.key_centroids.data_ptr(), st.value_centroids.data_ptr(), st.signs_left.data_ptr(),
                  st.signs_right.data_ptr(), flags, None, None, ns)
        ws = torch.empty(_lib.call("tq_decode_workspace_bytes", 1, cfg.kv_heads, hq, cfg.head_dim, ns, 0),
                         dtype=torch.uint8, device=hip_device)
        ref = torch.empty((1, hq, cfg.head_dim), dtype=torch.float32, device=hip_device)
        got = torch.full_like(ref, float("nan"))
        _lib.call("tq_decode", *common, ws.data_ptr(), ws.numel(), ref.data_ptr(), stream)
        _lib.call("tq_decode_noalloc", *common, got.data_ptr(), stream)
        torch.cuda.synchronize(hip_device)
        np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())


_FIRST_CALL_IN_CAPTURE = r"""
import sys
import numpy as np
import torch
import torque_hip as th
from torque_hip import _lib
from torque_hip._tensors import dtype_code

dev = torch.device("cuda", 0)
cfg = th.TorqueConfig(bit_width=4, head_dim=128, num_layers=1, kv_heads=2)
cache = th.TorqueKVCacheHIP(config=cfg, initial_capacity=2048, decode_tail_capacity=0)
gen = torch.Generator(device=dev).manual_seed(1)
cache.append_many(key=torch.randn((1, 2, 2048, 128), generator=gen, device=dev),
                  value=torch.randn((1, 2, 2048, 128), generator=gen, device=dev))
st = cache._store
q = torch.randn((1, 8, 128), generator=gen, device=dev)
out = torch.full((1, 8, 128), float("nan"), device=dev)
flags = _lib.TQ_ROTATE_QUERY | _lib.TQ_INVERSE_OUTPUT


def call():
    _lib.call("tq_decode_noalloc", q.data_ptr(), dtype_code(q), 1, 8, 2, 128, 4, st.key_codes.data_ptr(),
              st.value_codes.data_ptr(), st.capacity, st.length, st.key_centroids.data_ptr(),
              st.value_centroids.data_ptr(), st.signs_left.data_ptr(), st.signs_right.data_ptr(), flags, None, None,
              0, out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)


torch.cuda.synchronize()
print("first call inside a capture", flush=True)
graph = torch.cuda.CUDAGraph()
try:
    with torch.cuda.graph(graph):
        call()
except ValueError as e:
    assert "inside a stream capture" in str(e), e
    print("refused:", e, flush=True)
else:
    sys.exit("the first call inside a capture was not refused")
torch.cuda.synchronize()
call()  # eager: looks the scratch address up
torch.cuda.synchronize()
ref = out.clone()
assert torch.isfinite(ref).all()
out.fill_(float("nan"))
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    call()
for _ in range(3):
    out.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
print("ok", flush=True)
"""


def test_noalloc_first_call_inside_capture_is_refused(hip_device):
    """In a fresh process the first tq_decode_noalloc call on a device looks its scratch address up; made
    inside a stream capture it is refused with a message before anything is enqueued, and after one eager
    call the same call captures and replays."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    repo = Path(__file__).resolve().parents[1]
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(repo / "torque-mlx_amd"), str(repo), env.get("PYTHONPATH", "")])
    print("child: first tq_decode_noalloc call inside torch.cuda.graph", flush=True)
    proc = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE], env=env, capture_output=True, text=True,
                          timeout=110)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "refused:" in proc.stdout and proc.stdout.rstrip().endswith("ok"), proc.stdout
