"""The C-ABI library loads and exports every entry point include/torque_hip.h declares.

CPU only: nothing here launches a kernel (the calls below return before any
device work -- argument errors and pure host queries).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "torque_hip.h"


def _declared() -> dict[str, int]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(tq_[a-z_]+)\s*\(([^;{]*?)\)\s*;", text):
        args = m.group(2).strip()
        decls[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return decls


def test_header_declares_the_path():
    decls = _declared()
    for name in ("tq_fwht", "tq_quantize_pack", "tq_append", "tq_decode", "tq_decode_dense", "tq_last_error"):
        assert name in decls


def test_library_exports_every_declared_symbol():
    from torque_hip import _lib

    lib = ctypes.CDLL(str(_lib.library_path()))
    for name, nargs in _declared().items():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes binding"
        assert len(_lib.SIGNATURES[name][1]) == nargs, f"{name}: binding has {len(_lib.SIGNATURES[name][1])} args, header {nargs}"


def test_host_only_entry_points():
    from torque_hip import _lib

    lib = _lib.load()
    assert lib.tq_abi_version() == _lib.ABI_VERSION == 4
    # 4-bit rows in groups of 4 query heads: the f16-split matrix kernel, one 768-thread workgroup per CU
    assert lib.tq_decode_default_splits(1, 8, 32, 128, 4, 0, 32768, 256) == 32
    # the float32-product kernel (requested, or 3-bit rows): two 256-thread workgroups per CU
    assert lib.tq_decode_default_splits(1, 8, 32, 128, 4, 4, 32768, 256) == 64
    assert lib.tq_decode_default_splits(1, 8, 32, 128, 2, 0, 32768, 256) == 32  # 2-bit: the matrix kernel too
    assert lib.tq_decode_default_splits(1, 8, 32, 128, 3, 0, 32768, 256) == 64
    assert lib.tq_decode_default_splits(1, 8, 32, 128, 4, 0, 7, 256) == 1
    # a length cap just above one workgroup per CU drops to one per CU: 8192 + t tokens over 4 KV heads
    # would take 65 splits (260 workgroups), 8192 + 4096 tokens 96 (384, far enough over to keep)
    assert lib.tq_decode_default_splits(1, 4, 16, 256, 4, 0, 8192, 256) == 64
    assert lib.tq_decode_default_splits(1, 4, 16, 256, 4, 0, 8193, 256) == 64
    assert lib.tq_decode_default_splits(1, 4, 16, 256, 4, 0, 8192 + 4096, 256) == 96
    assert lib.tq_decode_default_splits(1, 8, 8, 64, 3, 0, 4096 + 64, 256) == 32  # 33 x 8 = 264 workgroups
    # head-group counts that do not divide the target round down, so no workgroup runs in a second wave:
    # 3 x 85 = 255 (matrix kernel, one per CU) and 3 x 170 = 510 (float32 kernel, two per CU)
    assert lib.tq_decode_default_splits(1, 3, 12, 128, 4, 0, 1 << 16, 256) == 85
    assert lib.tq_decode_default_splits(1, 3, 12, 128, 4, 4, 1 << 16, 256) == 170
    assert lib.tq_decode_default_splits(1, 5, 20, 128, 3, 0, 1 << 16, 256) == 102
    assert lib.tq_decode_workspace_bytes(1, 8, 32, 128, 64, 256) > 64 * 8 * 4 * 128 * 4
    assert lib.tq_decode_workspace_bytes(1, 8, 30, 128, 64, 256) == 0  # Hq not divisible
    mx, f32 = _lib.TQ_MATRIX_PRODUCTS, _lib.TQ_F32_PRODUCTS
    ks = lambda *a, **k: _lib.split_kernel(*a, num_cus=256, **k)
    # M: 256 blocks of 128 rows over 32 splits (8 per split): the matrix kernel
    assert ks(8, 32, 128, 4, 0, _lib.TQ_F16, 32768) == "decode_mx_kernel<128,true>"
    assert ks(8, 32, 64, 4, 0, _lib.TQ_F32, 32768) == "decode_mx_kernel<64,false>"
    assert ks(8, 32, 128, 4, f32, _lib.TQ_F16, 32768) == "decode_kernel<PackedB4,128,4>"
    assert ks(8, 32, 128, 2, 0, _lib.TQ_F16, 32768) == "decode_mx_kernel<128,true,2>"
    assert ks(8, 32, 128, 2, f32, _lib.TQ_F16, 32768) == "decode_kernel<PackedB2,128,4>"
    assert ks(8, 32, 64, 2, mx, _lib.TQ_F16, 32768) == "decode_kernel<PackedB2,64,4>"
    # head_dim 128 takes the matrix kernel from 4 blocks per split (16K tokens at 8 KV heads), not at 2
    assert ks(8, 32, 128, 4, 0, _lib.TQ_F16, 16384) == "decode_mx_kernel<128,true>"
    assert ks(8, 32, 128, 4, 0, _lib.TQ_F16, 8192) == "decode_kernel<PackedB4,128,4>"
    assert ks(8, 32, 128, 4, 0, _lib.TQ_F16, 8192, n_splits=16) == "decode_mx_kernel<128,true>"
    # head_dim 256 from 8: C4 (128K tokens, 2 KV heads) yes, a C5 layer (8K tokens, 4 KV heads) no
    assert ks(2, 8, 256, 4, 0, _lib.TQ_F16, 131072) == "decode_mx_kernel<256,true>"
    assert ks(2, 8, 256, 4, f32, _lib.TQ_F16, 131072) == "decode_kernel<PackedB4,256,4>"
    assert ks(4, 16, 256, 4, 0, _lib.TQ_F16, 8192) == "decode_kernel<PackedB4,256,4>"
    assert ks(4, 16, 256, 4, mx, _lib.TQ_F16, 8192) == "decode_mx_kernel<256,true>"
    assert ks(4, 16, 256, 4, mx, _lib.TQ_F16, 1, num_layers=24) == "decode_mx_kernel<256,true>"
    # 3 tokens per lane group (48-row iterations) where the 32-row deal leaves a nearly empty last iteration:
    # 8193..9216 rows over 64 splits (5 narrow against 3 wide), not 8192 (4 against 3), 9217 (73 splits: 4
    # against 3) or long sequences (forced float32 kernel at C4: 16 against 11)
    assert ks(4, 16, 256, 4, 0, _lib.TQ_F16, 8193) == "decode_kernel<PackedB4,256,4,3>"
    assert ks(4, 16, 256, 4, 0, _lib.TQ_F16, 9216) == "decode_kernel<PackedB4,256,4,3>"
    assert ks(4, 16, 256, 4, 0, _lib.TQ_F16, 9217) == "decode_kernel<PackedB4,256,4>"
    assert ks(4, 16, 256, 4, 0, _lib.TQ_F16, 8192) == "decode_kernel<PackedB4,256,4>"
    assert ks(4, 8, 256, 4, 0, _lib.TQ_F16, 8193) == "decode_kernel<PackedB4,256,2>"  # groups of 2: no such instance
    assert ks(4, 16, 256, 2, 0, _lib.TQ_F16, 8193) == "decode_kernel<PackedB2,256,4>"
    # groups of 2 and 3-bit rows never take it, forced or not
    assert ks(4, 8, 128, 4, mx, _lib.TQ_F16, 32768) == "decode_kernel<PackedB4,128,2>"
    assert ks(8, 32, 128, 3, mx, _lib.TQ_F16, 32768) == "decode_kernel<PackedB3,128,4>"
    with pytest.raises(ValueError):
        _lib.split_kernel(8, 30, 128, 4, 0, _lib.TQ_F16, 100)
    # the two product flags exclude each other in the host queries as in tq_decode
    with pytest.raises(ValueError, match="exclude each other"):
        _lib.split_kernel(8, 32, 128, 4, mx | f32, _lib.TQ_F16, 32768)
    assert lib.tq_decode_default_splits(1, 8, 32, 128, 4, mx | f32, 32768, 256) == _lib.TQ_ERR_BAD_ARG
    assert b"exclude each other" in lib.tq_last_error()


@pytest.mark.parametrize(
    ("args", "code", "message"),
    [
        (dict(head_dim=96), -2, "Unsupported head dimension: 96"),
        (dict(bits=5), -2, "Unsupported bit width: 5"),
        (dict(query_heads=30), -1, "must be divisible by kv_heads"),
        (dict(capacity=5), -1, "capacity must be >= seq_len"),
    ],
)
def test_decode_argument_errors(args, code, message):
    from torque_hip import _lib

    lib = _lib.load()
    p = dict(head_dim=128, bits=4, query_heads=32, capacity=10)
    p.update(args)
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    rc = lib.tq_decode(fake, 0, 1, p["query_heads"], 8, p["head_dim"], p["bits"], fake, fake, p["capacity"], 10,
                       fake, fake, None, None, 0, None, None, 0, fake, 1 << 30, fake, None)
    assert rc == code
    assert message in lib.tq_last_error().decode()


def test_last_error_is_per_thread():
    """tq_last_error() is thread-local: two threads that fail differently at the same moment each read
    back their own message (validation runs on the host before any launch, so no GPU is needed)."""
    import threading

    from torque_hip import _lib

    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    barrier = threading.Barrier(2, timeout=30)  # a thread that dies breaks it instead of hanging the other
    seen: dict[int, list[str]] = {96: [], 5: []}

    def run(head_dim, bits, key):
        for _ in range(50):
            rc = lib.tq_decode(fake, 0, 1, 32, 8, head_dim, bits, fake, fake, 10, 10, fake, fake, None, None, 0,
                               None, None, 0, fake, 1 << 30, fake, None)
            assert rc == -2
            barrier.wait()  # both threads have set their error before either reads it
            seen[key].append(lib.tq_last_error().decode())
            barrier.wait()

    threads = [threading.Thread(target=run, args=(96, 4, 96)), threading.Thread(target=run, args=(128, 5, 5))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert len(seen[96]) == len(seen[5]) == 50
    assert all("Unsupported head dimension: 96" in m for m in seen[96])
    assert all("Unsupported bit width: 5" in m for m in seen[5])


@pytest.mark.parametrize(
    ("num_layers", "seq_len", "n_splits", "message"),
    [
        (1 << 22, 10, 0, "exceeds one launch"),  # 2^25 (layer, head group) units > 2^24 workgroups
        (1 << 19, 100_000, 8, "exceeds one merge launch"),  # 2^19 x 32 heads x 4 merge groups > 2^24
    ],
)
def test_decode_launch_size_errors(num_layers, seq_len, n_splits, message):
    from torque_hip import _lib

    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    rc = lib.tq_decode(fake, 0, num_layers, 32, 8, 128, 4, fake, fake, seq_len, seq_len, fake, fake, None, None, 0,
                       None, None, n_splits, fake, 1 << 62, fake, None)
    assert rc == -1
    assert message in lib.tq_last_error().decode()


def _decode_args(fake, n_splits, ws_bytes):
    # tq_decode at the metric shape (1 layer, 32 query / 8 KV heads, D=128, 4-bit, 32K tokens)
    return (fake, 0, 1, 32, 8, 128, 4, fake, fake, 32768, 32768, fake, fake, None, None, 0, None, None, n_splits, fake,
            ws_bytes, fake, None)


@pytest.mark.parametrize("n_splits", [1, 17, 64, 256])
def test_decode_rejects_short_workspace(n_splits):
    """A workspace sized below what the resolved split plan needs is refused before any launch."""
    from torque_hip import _lib

    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    need = lib.tq_decode_workspace_bytes(1, 8, 32, 128, n_splits, 256)
    assert need > 0
    rc = lib.tq_decode(*_decode_args(fake, n_splits, need - 1))
    assert rc == -1
    assert f"smaller than the {need} bytes this call needs ({n_splits} splits)" in lib.tq_last_error().decode()
    # the same short workspace for the other decode entry points
    rc = lib.tq_decode_dense(fake, 0, fake, fake, 1, 1, 32, 8, 128, 32768, 32768, None, None, 0, n_splits, fake,
                             need - 1, fake, None)
    assert rc == -1 and "bytes this call needs" in lib.tq_last_error().decode()
    rc = lib.tq_decode_scaled(fake, 0, 1, 32, 8, 128, 4, fake, fake, fake, fake, 32768, 32768, fake, fake, None, None,
                              0, None, None, n_splits, fake, need - 1, fake, None)
    assert rc == -1 and "bytes this call needs" in lib.tq_last_error().decode()
    rc = lib.tq_decode_append(fake, 0, fake, fake, 0, 1, 32, 8, 128, 4, fake, fake, 32769, 32768, fake, fake, fake,
                              fake, fake, fake, 3, 3, n_splits, fake, need - 1, fake, None)
    assert rc == -1 and "bytes this call needs" in lib.tq_last_error().decode()


def test_workspace_query_covers_default_plan():
    """n_splits <= 0 sizes the workspace for the default split count at any sequence length."""
    from torque_hip import _lib

    lib = _lib.load()
    for seq_len in (1, 100, 4096, 32768, 1 << 20):
        ns = max(lib.tq_decode_default_splits(1, 8, 32, 128, bits, 0, seq_len, 256) for bits in (0, 2, 3, 4))
        assert lib.tq_decode_workspace_bytes(1, 8, 32, 128, ns, 256) <= lib.tq_decode_workspace_bytes(1, 8, 32, 128, 0,
                                                                                                        256)


def test_decode_append_rejects_bad_kv_dtype():
    from torque_hip import _lib

    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    rc = lib.tq_decode_append(fake, 0, fake, fake, 7, 1, 32, 8, 128, 4, fake, fake, 32769, 32768, fake, fake, fake,
                              fake, fake, fake, 3, 3, 0, fake, 1 << 30, fake, None)
    assert rc == -1 and "new key/value dtype" in lib.tq_last_error().decode()


def test_status_mapping():
    from torque_hip import _lib

    _lib.load()
    with pytest.raises(ValueError, match="Unsupported bit width"):
        _lib.call("tq_quantize_pack", 0x1000, 4, 64, 7, 0x1000, 0x1000, None)
