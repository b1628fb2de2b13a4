"""The C ABI library loads and exports every entry point include/laya_hip.h declares (no GPU)."""
import ctypes as ct
import re
from pathlib import Path

import numpy as np
import pytest

from laya_cuda import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "laya_hip.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t|const char\*)\s+(laya_\w+)\(", text, re.M)))


def test_header_declares_the_boundary():
    names = declared()
    for name in ("laya_create", "laya_load_weight", "laya_finalize", "laya_predict", "laya_destroy",
                 "laya_last_error", "laya_op_attention", "laya_op_linear"):
        assert name in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [name for name in declared() if not hasattr(lib, name)]
    assert not missing
    assert set(declared()) <= set(_lib.SIGNATURES)
    assert lib.laya_abi_version() == _lib.ABI_VERSION == 2


def test_library_links_no_gemm_library():
    """Every projection runs on this library's own MFMA kernels: no BLAS library is linked into
    liblaya_hip.so or referenced by its dynamic symbol table."""
    import subprocess
    path = Path(_lib.__file__).resolve().parent / "liblaya_hip.so"
    symbols = subprocess.run(["nm", "-D", str(path)], check=True, capture_output=True, text=True).stdout
    needed = subprocess.run(["readelf", "-d", str(path)], check=True, capture_output=True, text=True).stdout
    for text in (symbols, needed):
        assert not re.search(r"hipblas|rocblas|cublas", text, re.I)


def test_binding_refuses_a_library_of_another_abi_version(monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)  # force a fresh load
    monkeypatch.setattr(_lib, "ABI_VERSION", _lib.ABI_VERSION + 1)
    with pytest.raises(RuntimeError, match="ABI version"):
        _lib.load()
    assert _lib._lib is None  # nothing half-loaded is cached


def test_binding_reports_the_version_of_a_library_missing_exports(monkeypatch):
    """A library of another ABI that lacks the other exports fails on its version, not on a
    missing symbol: the version is bound and compared before anything else is typed."""
    def version():
        return _lib.ABI_VERSION + 7

    class OtherAbi:  # exports laya_abi_version only
        laya_abi_version = staticmethod(version)

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib.ct, "CDLL", lambda path: OtherAbi())
    with pytest.raises(RuntimeError, match=f"ABI version {_lib.ABI_VERSION + 7}"):
        _lib.load()
    assert _lib._lib is None


def test_packed_block_size_matches_the_python_packer():
    from laya_cuda.runtime import pack
    lib = _lib.load()
    for m, b, k in [(96, 1, 8), (512, 2, 8), (16384, 128, 128)]:
        shape = _lib.LayaShape(m, b, k)
        seqs = [np.full(20, 7, np.int32)]
        block = pack(seqs, [(0, [1, 2], 1)], (m, b, k), pad=0)
        assert lib.laya_packed_ints(ct.byref(shape)) == block.size
    assert lib.laya_packed_ints(ct.byref(_lib.LayaShape(0, 1, 8))) == -1


def tiles(starts, lengths, m, block, max_tiles=None):
    lib = _lib.load()
    max_tiles = max_tiles or m // 16
    out = np.full(4 * max_tiles, 7, np.int32)
    s, n = np.asarray(starts, np.int32), np.asarray(lengths, np.int32)
    count = lib.laya_attention_tiles(s.ctypes.data_as(ct.POINTER(ct.c_int32)), n.ctypes.data_as(ct.POINTER(ct.c_int32)),
                                     len(s), m, block, out.ctypes.data_as(ct.POINTER(ct.c_int32)), max_tiles)
    quads = out.reshape(-1, 4)
    if count >= 0:  # every entry past the used ones is an empty range
        assert (quads[count:, 0] == quads[count:, 1]).all() and (quads[count:, 3] == -1).all()
    return count, quads[:max(count, 0)]


@pytest.mark.parametrize("block", [32, 64, 128])
def test_attention_tiles_cover_every_row_once(block):
    lengths = [250, 131, 1, 16, 500]
    starts, at = [], 0
    for n in lengths:
        starts.append(at)
        at += -(-n // 16) * 16
    m = at + 64
    count, t = tiles(starts, lengths, m, block)
    assert count > 0
    covered = np.zeros(m, int)
    for r0, r1, kstart, klen in t:
        assert 0 < r1 - r0 <= block
        covered[r0:r1] += 1
        if klen >= 0:  # a tile never straddles a sequence's span, and carries that sequence's keys
            seq = starts.index(kstart)
            assert klen == lengths[seq]
            assert kstart <= r0 and r1 <= kstart + -(-klen // 16) * 16
    assert (covered == 1).all()
    assert (t[:, 3] == -1).sum() >= 1  # rows past the last sequence are zero tiles


def test_attention_tiles_reject_bad_layouts():
    assert tiles([8], [10], 64, 64)[0] == -1            # not 16-aligned
    assert tiles([0, 0], [16, 16], 64, 64)[0] == -1     # overlapping
    assert tiles([0], [100], 64, 64)[0] == -1           # past the slot
    assert tiles([0], [64], 64, 16, max_tiles=2)[0] == -1  # tile list too small


def test_create_without_gpu_reports_an_error():
    """On a machine without a usable gfx950 device, create fails with a message, not a crash."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = _lib.load()
    cfg = _lib.LayaConfig(width=64, heads=1, layers=1, intermediate=256, vocab=10, max_positions=16, type_vocab=2,
                          norm_order=0, pos_kind=0, ffn_kind=0, bias=1, eps=1e-12, window=-1, global_every=1,
                          head_layers=0, n_act=2, act_hidden=256, max_len=16, mfma_dtype=_lib.F16)
    handle = ct.c_void_p()
    rc = lib.laya_create(ct.byref(cfg), 0, 4, ct.byref(handle))
    assert rc != 0 and not handle.value
    assert _lib.error(None)


def test_create_rejects_unbuilt_variants_before_touching_the_device():
    """Only the two built variants pass: BERT-style and the reference's ModernBERT executor.  A mix
    (pre-LN with learned positions) or a ModernBERT config without RoPE thetas is rejected."""
    lib = _lib.load()
    cfg = _lib.LayaConfig(width=64, heads=1, layers=1, intermediate=256, vocab=10, max_positions=16, type_vocab=2,
                          norm_order=1, pos_kind=0, ffn_kind=1, bias=0, eps=1e-5, window=64, global_every=3,
                          head_layers=1, n_act=2, act_hidden=256, max_len=16, mfma_dtype=_lib.F16,
                          theta_global=160000.0, theta_local=10000.0)
    handle = ct.c_void_p()
    assert lib.laya_create(ct.byref(cfg), 0, 4, ct.byref(handle)) == _lib.EINVAL
    assert "variant not built" in _lib.error(None)
    cfg.pos_kind, cfg.theta_local = 1, 0.0
    assert lib.laya_create(ct.byref(cfg), 0, 4, ct.byref(handle)) == _lib.EINVAL
    assert "variant not built" in _lib.error(None)
    cfg.norm_order, cfg.pos_kind, cfg.ffn_kind, cfg.bias, cfg.window, cfg.head_layers = 0, 0, 0, 1, -1, 0
    cfg.heads = 2  # width != heads * 64
    assert lib.laya_create(ct.byref(cfg), 0, 4, ct.byref(handle)) == _lib.EINVAL
    assert "64-wide" in _lib.error(None)


def test_attention_block_rows_per_mode():
    """Query rows per tile: shared K/V 32 x waves, split keys 32, paired query groups 64; -1 for
    pairs a kernel does not exist for."""
    lib = _lib.load()
    assert [lib.laya_attention_block(0, w) for w in (1, 2, 4, 8, 3)] == [32, 64, 128, 256, -1]
    assert [lib.laya_attention_block(1, w) for w in (1, 2, 4, 8)] == [-1, 32, 32, 32]
    assert [lib.laya_attention_block(2, w) for w in (2, 4, 8)] == [-1, 64, 64]
    assert lib.laya_attention_block(3, 4) == -1


def test_device_queries():
    """laya_device_count reports zero devices (not an error) without a GPU; laya_device_info
    refuses a device that does not exist."""
    lib = _lib.load()
    count = ct.c_int(-1)
    assert lib.laya_device_count(ct.byref(count)) == _lib.OK and count.value >= 0
    info = _lib.LayaDevice()
    assert lib.laya_device_info(count.value, ct.byref(info)) != _lib.OK
    assert "no HIP device" in _lib.error(None)
    if count.value:
        assert lib.laya_device_info(0, ct.byref(info)) == _lib.OK
        assert info.hbm_bytes > 0 and info.compute_units > 0 and info.free_bytes <= info.hbm_bytes


def test_stage_queries_without_a_handle():
    lib = _lib.load()
    names = [lib.laya_stage_name(i).decode() for i in range(lib.laya_stage_count())]
    assert names[0] == "embed_norm" and "attention" in names and "head_qkv" in names
    assert lib.laya_stage_name(len(names)) is None
    n, first = ct.c_int32(), ct.c_int32()
    assert lib.laya_stage_launches(None, 0, ct.byref(n), ct.byref(first)) == _lib.EINVAL
