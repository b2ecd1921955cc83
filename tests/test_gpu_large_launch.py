"""Row kernels on calls larger than one launch.

The rotation, append (rotate, quantize, pack) and unpack entry points cut a
call into launches of at most 2^20 workgroups (a HIP launch holds at most
2^32 - 1 work-items): at whole (layer, head) groups, or at token ranges when
one group alone is larger.  Each case here crosses that size and is checked
bit-exact against the same work done by several smaller calls that each fit
one launch (cut at other points), and against the CPU oracle on the rows
around every cut.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import torque_oracle as o

pytestmark = pytest.mark.gpu

MAX_BLOCKS = 1 << 20  # workgroups per launch of the row kernels
WAVES = 4  # wavefronts per workgroup
D = 64


def _p(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _signs(seed: int) -> tuple[torch.Tensor, torch.Tensor, np.ndarray, np.ndarray]:
    sl, sr = o.rotation_signs_from_seed(D, seed)
    return torch.from_numpy(sl).cuda(), torch.from_numpy(sr).cuda(), sl, sr


def _near(cuts: list[int], total: int, width: int = 3) -> np.ndarray:
    rows = {0, total - 1}
    for c in cuts:
        rows.update(range(max(0, c - width), min(total, c + width)))
    return np.array(sorted(rows))


def test_fwht_past_one_launch(hip_device):
    from torque_hip import _lib

    rows = MAX_BLOCKS * WAVES + 1000  # one wavefront per row: two launches
    gen = torch.Generator(device=hip_device).manual_seed(3)
    x = torch.randn(rows, D, device=hip_device, dtype=torch.float16, generator=gen)
    sl_t, sr_t, sl, sr = _signs(5)
    y = torch.empty(rows, D, device=hip_device, dtype=torch.float32)
    _lib.call("tq_fwht", _p(x), _lib.TQ_F16, _p(y), rows, D, _p(sl_t), _p(sr_t), 0, _stream())
    parts = torch.empty_like(y)
    cut = 1_234_567
    for r0, r1 in ((0, cut), (cut, rows)):
        _lib.call("tq_fwht", _p(x[r0:r1]), _lib.TQ_F16, _p(parts[r0:r1]), r1 - r0, D, _p(sl_t), _p(sr_t), 0, _stream())
    torch.cuda.synchronize()
    assert torch.equal(y, parts)
    idx = _near([MAX_BLOCKS * WAVES, cut], rows)
    exp = o.rotation_apply(x[idx].float().cpu().numpy(), sl, sr)
    np.testing.assert_array_equal(y[idx].cpu().numpy(), exp)


def _append(keys, values, codes_k, codes_v, *, kv_heads, seq_new, capacity, offset, bnd, sl_t, sr_t, bits):
    from torque_hip import _lib

    _lib.call(
        "tq_append", _p(keys), _p(values), _lib.TQ_F16, 1, kv_heads, seq_new, D, bits, _p(sl_t), _p(sr_t),
        _lib.TQ_ROTATE_KEYS | _lib.TQ_ROTATE_VALUES, _p(bnd), _p(bnd), _p(codes_k), _p(codes_v), capacity, offset,
        _stream(),
    )


def _oracle_words(x_rows: np.ndarray, sl, sr, bnd: np.ndarray, bits: int) -> np.ndarray:
    rot = o.rotation_apply(x_rows.astype(np.float32), sl, sr)
    return o.pack_indices_batched(o.quantize_boundary_count(rot, bnd), bits)


@pytest.mark.parametrize(
    ("kv_heads", "seq_new"),
    [
        (1, MAX_BLOCKS * WAVES // 2 + 37),  # one group larger than a launch: cut at tokens
        (5, 1_000_000),  # two groups per launch: cut at groups
    ],
)
def test_append_past_one_launch(hip_device, kv_heads, seq_new):
    bits = 3
    W = o.packed_words_for_head_dim(D, bits)
    offset, capacity = 3, seq_new + 8
    gen = torch.Generator(device=hip_device).manual_seed(11)
    keys = torch.randn(kv_heads, seq_new, D, device=hip_device, dtype=torch.float16, generator=gen)
    values = torch.randn(kv_heads, seq_new, D, device=hip_device, dtype=torch.float16, generator=gen) * 0.5
    sl_t, sr_t, sl, sr = _signs(9)
    bnd_np = o.codebook_boundaries(o.build_gaussian_codebook(bits, seed=bits))
    bnd = torch.from_numpy(bnd_np).cuda()
    kc = torch.zeros(kv_heads, capacity, W, device=hip_device, dtype=torch.int32)
    vc = torch.zeros_like(kc)
    _append(keys, values, kc, vc, kv_heads=kv_heads, seq_new=seq_new, capacity=capacity, offset=offset, bnd=bnd,
            sl_t=sl_t, sr_t=sr_t, bits=bits)
    # The same rows, one head at a time and cut at another token, each call one launch.
    kp, vp = torch.zeros_like(kc), torch.zeros_like(vc)
    cut = 600_001
    for h in range(kv_heads):
        for t0, t1 in ((0, cut), (cut, seq_new)):
            _append(keys[h, t0:t1], values[h, t0:t1], kp[h], vp[h], kv_heads=1, seq_new=t1 - t0, capacity=capacity,
                    offset=offset + t0, bnd=bnd, sl_t=sl_t, sr_t=sr_t, bits=bits)
    torch.cuda.synchronize()
    assert torch.equal(kc, kp) and torch.equal(vc, vp)
    assert not kc[:, :offset].any() and not kc[:, offset + seq_new :].any()
    max_rows = MAX_BLOCKS * WAVES // 2
    cuts = [max_rows, cut] if kv_heads == 1 else [cut]
    idx = _near(cuts, seq_new)
    for h in {0, kv_heads - 1}:
        for src, dst in ((keys, kc), (values, vc)):
            exp = _oracle_words(src[h, idx].float().cpu().numpy(), sl, sr, bnd_np, bits)
            got = dst[h, offset + idx].cpu().numpy().view(np.uint32)
            np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize(
    ("groups", "seq_len"),
    [
        (1, MAX_BLOCKS * 256 // D + 11),  # one thread per value: cut at tokens
        (3, 2_000_000),  # two groups per launch: cut at groups
    ],
)
def test_unpack_past_one_launch(hip_device, groups, seq_len):
    from torque_hip import _lib

    bits = 4
    W = o.packed_words_for_head_dim(D, bits)
    capacity = seq_len + 5
    gen = torch.Generator(device=hip_device).manual_seed(17)
    codes = torch.randint(-(2**31), 2**31 - 1, (groups, capacity, W), device=hip_device, dtype=torch.int32,
                          generator=gen)
    cent_np = o.build_gaussian_codebook(bits, seed=1)
    cent = torch.from_numpy(cent_np).cuda()
    out = torch.empty(groups, seq_len, D, device=hip_device, dtype=torch.float32)
    _lib.call("tq_unpack_dequantize", _p(codes), groups, capacity, seq_len, D, bits, _p(cent), _p(out), _stream())
    parts = torch.empty_like(out)
    cut = 1_700_003
    for g in range(groups):
        for t0, t1 in ((0, cut), (cut, seq_len)):
            _lib.call("tq_unpack_dequantize", _p(codes[g, t0:]), 1, capacity, t1 - t0, D, bits, _p(cent),
                      _p(parts[g, t0:t1]), _stream())
    torch.cuda.synchronize()
    assert torch.equal(out, parts)
    max_tokens = MAX_BLOCKS * 256 // D
    cuts = [max_tokens, cut] if groups == 1 else [cut]
    idx = _near(cuts, seq_len)
    for g in {0, groups - 1}:
        words = codes[g, idx].cpu().numpy().view(np.uint32)
        exp = o.dequantize(o.unpack_indices_batched(words, bits, D), cent_np)
        np.testing.assert_array_equal(out[g, idx].cpu().numpy(), exp)
