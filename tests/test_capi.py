"""The C ABI library: loads, exports every declared symbol, rejects bad arguments (CPU only —
every call here fails validation or is a no-op before any GPU work)."""

import ctypes
import os
import re

import pytest

from mlx_tree_spec_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qmm4.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(\w+)\s*\(", src, flags=re.M)))


def test_header_declares_expected_api():
    assert declared_functions() == sorted(["qmm4_affine_bf16", "qmm4_affine_bf16_noalloc", "qmm4_gate_up_silu_bf16",
                                           "dequant4_affine_bf16", "qmm4_add_rms_norm_bf16",
                                           "qmm4_add_rms_norm_qmm_bf16", "qmm4_last_error", "qmm4_abi_version"])


def test_constants_match_the_header():
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    defines = {k: v for k, v in re.findall(r"^#define\s+(QMM4_\w+)\s+(.+?)\s*$", src, flags=re.M)}
    for name in ("QMM4_OK", "QMM4_ERR_INVALID", "QMM4_ERR_UNSUPPORTED", "QMM4_ERR_NOMEM", "QMM4_ERR_HIP",
                 "QMM4_ERR_CAPTURE", "QMM4_EPILOGUE_NONE", "QMM4_EPILOGUE_SILU_MUL", "QMM4_NOALLOC_SCRATCH_BYTES"):
        assert name in defines, name
        value = eval(defines[name].replace("u", ""), {})  # integer literals and products
        assert getattr(_lib, name) == value, (name, defines[name])


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES
    assert lib.qmm4_abi_version() == 1


def call(M=4, N=32, K=128, gs=64, bits=4, transpose=1, ptr=0x10000, y=0x20000):
    lib = _lib.load()
    return lib.qmm4_affine_bf16(ptr, ptr, ptr, ptr, y, M, N, K, gs, bits, transpose, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(bits=3), _lib.QMM4_ERR_UNSUPPORTED, "bits=3"),
    (dict(bits=8), _lib.QMM4_ERR_UNSUPPORTED, "bits=8"),
    (dict(gs=32), _lib.QMM4_ERR_UNSUPPORTED, "group_size=32"),
    (dict(gs=128), _lib.QMM4_ERR_UNSUPPORTED, "group_size=128"),
    (dict(transpose=0), _lib.QMM4_ERR_UNSUPPORTED, "transpose=0"),
    (dict(K=192), _lib.QMM4_ERR_INVALID, "K=192"),
    (dict(K=0), _lib.QMM4_ERR_INVALID, "invalid shape"),
    (dict(N=24), _lib.QMM4_ERR_INVALID, "N=24"),
    (dict(M=-1), _lib.QMM4_ERR_INVALID, "invalid shape"),
    (dict(M=1 << 31), _lib.QMM4_ERR_INVALID, "exceeds"),
    (dict(ptr=0), _lib.QMM4_ERR_INVALID, "null pointer"),
    (dict(ptr=0x10008), _lib.QMM4_ERR_INVALID, "16-byte aligned"),
    (dict(y=0x20001), _lib.QMM4_ERR_INVALID, "2-byte aligned"),
])
def test_qmm_rejects(kw, code, msg):
    assert call(**kw) == code
    assert msg in _lib.last_error()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(bits=8), _lib.QMM4_ERR_UNSUPPORTED, "bits=8"),
    (dict(K=192), _lib.QMM4_ERR_INVALID, "K=192"),
    (dict(ptr=0x10008), _lib.QMM4_ERR_INVALID, "16-byte aligned"),
])
def test_noalloc_rejects_like_qmm(kw, code, msg):
    """The no-allocation entry point makes the same checks before touching the device."""
    lib = _lib.load()
    a = dict(M=4, N=32, K=128, gs=64, bits=4, transpose=1, ptr=0x10000, y=0x20000)
    a.update(kw)
    rc = lib.qmm4_affine_bf16_noalloc(a["ptr"], a["ptr"], a["ptr"], a["ptr"], a["y"], a["M"], a["N"], a["K"],
                                      a["gs"], a["bits"], a["transpose"], None)
    assert rc == code
    assert msg in _lib.last_error()


def test_qmm_empty_is_noop():
    assert call(M=0, ptr=0) == _lib.QMM4_OK
    assert call(N=0, ptr=0) == _lib.QMM4_OK
    assert _lib.last_error() == ""


def call_gate_up(M=4, N=64, K=128, gs=64, bits=4, transpose=1, ptr=0x10000, y=0x20000):
    lib = _lib.load()
    return lib.qmm4_gate_up_silu_bf16(ptr, ptr, ptr, ptr, y, M, N, K, gs, bits, transpose, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(bits=2), _lib.QMM4_ERR_UNSUPPORTED, "bits=2"),
    (dict(gs=128), _lib.QMM4_ERR_UNSUPPORTED, "group_size=128"),
    (dict(transpose=0), _lib.QMM4_ERR_UNSUPPORTED, "transpose=0"),
    (dict(K=64), _lib.QMM4_ERR_INVALID, "K=64"),
    (dict(N=48), _lib.QMM4_ERR_INVALID, "multiple of 32"),
    (dict(N=24), _lib.QMM4_ERR_INVALID, "N=24"),
    (dict(ptr=0), _lib.QMM4_ERR_INVALID, "null pointer"),
    (dict(y=0x20008), _lib.QMM4_ERR_INVALID, "y must be 16-byte aligned"),
])
def test_gate_up_rejects(kw, code, msg):
    assert call_gate_up(**kw) == code
    assert msg in _lib.last_error()


@pytest.mark.parametrize("rows,d,eps,ptr,msg", [
    (4, 12, 1e-6, 0x10000, "multiple of 8"),
    (4, 0, 1e-6, 0x10000, "invalid shape"),
    (4, 16392, 1e-6, 0x10000, "at most 16384"),
    (-1, 64, 1e-6, 0x10000, "invalid shape"),
    (4, 64, -1.0, 0x10000, "eps"),
    (4, 64, float("nan"), 0x10000, "eps"),
    (4, 64, 1e-6, 0, "null pointer"),
    (4, 64, 1e-6, 0x10008, "16-byte aligned"),
])
def test_add_rms_norm_rejects(rows, d, eps, ptr, msg):
    lib = _lib.load()
    assert lib.qmm4_add_rms_norm_bf16(ptr, ptr, ptr, ptr, ptr, rows, d, eps, None) == _lib.QMM4_ERR_INVALID
    assert msg in _lib.last_error()


def test_add_rms_norm_empty_is_noop():
    assert _lib.load().qmm4_add_rms_norm_bf16(0, 0, 0, 0, 0, 0, 64, 1e-6, None) == _lib.QMM4_OK


def call_norm_qmm(M=2, N=64, K=128, eps=1e-6, epilogue=0, gs=64, bits=4, x=0x100000, r=0x200000, nw=0x300000,
                  h=0x400000, n=0x500000, w=0x600000, y=0x700000):
    lib = _lib.load()
    return lib.qmm4_add_rms_norm_qmm_bf16(x, r, nw, eps, h, n, w, w, w, y, M, N, K, gs, bits, 1, epilogue, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(bits=8), _lib.QMM4_ERR_UNSUPPORTED, "bits=8"),
    (dict(K=192), _lib.QMM4_ERR_INVALID, "K=192"),
    (dict(N=24), _lib.QMM4_ERR_INVALID, "N=24"),
    (dict(K=16512), _lib.QMM4_ERR_INVALID, "largest row"),
    (dict(epilogue=2), _lib.QMM4_ERR_INVALID, "epilogue=2"),
    (dict(epilogue=1, N=48), _lib.QMM4_ERR_INVALID, "multiple of 32"),
    (dict(eps=-1.0), _lib.QMM4_ERR_INVALID, "eps"),
    (dict(eps=float("inf")), _lib.QMM4_ERR_INVALID, "eps"),
    (dict(r=0), _lib.QMM4_ERR_INVALID, "null pointer"),
    (dict(h=0), _lib.QMM4_ERR_INVALID, "null pointer"),
    (dict(n=0x500008), _lib.QMM4_ERR_INVALID, "16-byte aligned"),
    (dict(nw=0x300004), _lib.QMM4_ERR_INVALID, "16-byte aligned"),
    (dict(epilogue=1, y=0x700002), _lib.QMM4_ERR_INVALID, "y must be 16-byte aligned"),
    (dict(h=0x100000), _lib.QMM4_ERR_INVALID, "overlap x, r, weight"),            # h on x
    (dict(n=0x200000 + 256), _lib.QMM4_ERR_INVALID, "overlap x, r, weight"),      # n inside r
    (dict(y=0x300000 + 64), _lib.QMM4_ERR_INVALID, "overlap x, r, weight"),       # y inside weight
    (dict(h=0x600000 + 128), _lib.QMM4_ERR_INVALID, "overlap x, r, weight"),      # h inside w
    (dict(n=0x400000 + 496), _lib.QMM4_ERR_INVALID, "overlap each other"),        # n's first row on h's last bytes
    (dict(y=0x500000), _lib.QMM4_ERR_INVALID, "overlap each other"),
])
def test_norm_qmm_rejects(kw, code, msg):
    """Every check of the folded norm + projection, before any device work (M=2, K=128: 512-byte rows)."""
    assert call_norm_qmm(**kw) == code
    assert msg in _lib.last_error()


def test_norm_qmm_empty_is_noop():
    assert call_norm_qmm(M=0, x=0, r=0, nw=0, h=0, n=0, w=0, y=0) == _lib.QMM4_OK
    assert _lib.last_error() == ""


def test_gate_up_empty_is_noop():
    assert call_gate_up(M=0, ptr=0) == _lib.QMM4_OK
    assert call_gate_up(N=0, ptr=0) == _lib.QMM4_OK


def test_dequant_rejects():
    lib = _lib.load()
    p = 0x10000
    assert lib.dequant4_affine_bf16(p, p, p, p, 8, 96, 64, 4, None) == _lib.QMM4_ERR_INVALID
    assert "K" in _lib.last_error()
    for gs, bits in ((64, 3), (64, 5), (64, 6), (64, 16), (16, 4), (256, 8)):
        assert lib.dequant4_affine_bf16(p, p, p, p, 8, 256, gs, bits, None) == _lib.QMM4_ERR_UNSUPPORTED
        assert (f"bits={bits}" if bits not in (2, 4, 8) else f"group_size={gs}") in _lib.last_error()
    # K must be whole groups of the format's group size.
    assert lib.dequant4_affine_bf16(p, p, p, p, 8, 96, 32 * 2, 8, None) == _lib.QMM4_ERR_INVALID
    assert lib.dequant4_affine_bf16(p, p, p, p, 8, 64, 128, 2, None) == _lib.QMM4_ERR_INVALID
    assert lib.dequant4_affine_bf16(0, p, p, p, 8, 128, 64, 4, None) == _lib.QMM4_ERR_INVALID
    assert lib.dequant4_affine_bf16(p + 4, p, p, p, 8, 128, 64, 4, None) == _lib.QMM4_ERR_INVALID
    assert lib.dequant4_affine_bf16(0, 0, 0, 0, 0, 128, 64, 4, None) == _lib.QMM4_OK


def test_error_message_is_thread_local():
    import threading

    assert call(bits=3) == _lib.QMM4_ERR_UNSUPPORTED
    seen = []
    t = threading.Thread(target=lambda: seen.append(_lib.last_error()))
    t.start()
    t.join()
    assert seen == [""] and "bits=3" in _lib.last_error()


def test_check_maps_codes():
    call(bits=3)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.QMM4_ERR_UNSUPPORTED, "t")
    with pytest.raises(ValueError):
        _lib.check(_lib.QMM4_ERR_INVALID, "t")
    with pytest.raises(MemoryError):
        _lib.check(_lib.QMM4_ERR_NOMEM, "t")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.QMM4_ERR_HIP, "t")
    _lib.check(_lib.QMM4_OK, "t")
