"""C-ABI checks that need no GPU: the library loads, exports every entry point declared in
include/orator_attn.h, and rejects bad arguments before any launch."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

from orator_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols() -> list[str]:
    names = []
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names += re.findall(r"^(?:int|const char\*)\s+(orator_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_signatures_cover_header():
    names = set(declared_symbols()) - {"orator_last_error"}
    assert names == set(_lib.SIGNATURES), names ^ set(_lib.SIGNATURES)


def test_version():
    assert _lib.lib().orator_version() >= 1


# Validation runs before any HIP call, so these work without a device.
FAKE = 0x1000  # never dereferenced: every call below is rejected first


def test_nonpositive_sizes_are_noops():
    lib = _lib.lib()
    assert lib.orator_rms_norm(None, None, None, 0, 128, 1e-6, None) == _lib.ORATOR_OK
    assert lib.orator_swiglu(None, None, None, 0, None) == _lib.ORATOR_OK
    assert lib.orator_rope_half(None, None, 0, 16, 128, 1e6, None) == _lib.ORATOR_OK
    assert lib.orator_gqa_decode(None, None, None, None, 0, 8, 128, None, 16, 0.1,
                                 None) == _lib.ORATOR_OK
    assert lib.orator_kv_write(None, None, None, None, 0, 8, 128, None, 16,
                               None) == _lib.ORATOR_OK


def test_null_pointers_rejected():
    lib = _lib.lib()
    rc = lib.orator_rms_norm(None, FAKE, FAKE, 4, 128, 1e-6, None)
    assert rc == _lib.ORATOR_ERR_INVALID
    assert b"null" in lib.orator_last_error()


def test_unsupported_decode_shapes_rejected():
    lib = _lib.lib()
    args = (FAKE, FAKE, FAKE, FAKE)
    # any head size up to 1024 and any group run (the generic kernel); past 1024 is rejected
    assert lib.orator_gqa_decode(*args, 16, 8, 2048, FAKE, 64, 0.1, None) == _lib.ORATOR_ERR_UNSUPPORTED
    assert lib.orator_gqa_prefill(*args, 4, 16, 8, 1032, FAKE, 64, 0.1,
                                  None) == _lib.ORATOR_ERR_UNSUPPORTED
    # Hq not a multiple of Hkv
    assert lib.orator_gqa_decode(*args, 12, 8, 128, FAKE, 64, 0.1, None) == _lib.ORATOR_ERR_INVALID
    # QK-norm folding: Dh 128 and groups {1, 2, 4} only
    assert lib.orator_gqa_decode_append_qknorm(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64, 8, 128,
                                               FAKE, 64, 0.1, FAKE, FAKE, 1e-6, FAKE, 64,
                                               None) == _lib.ORATOR_ERR_UNSUPPORTED
    # paged: page size must be a power of two >= 16
    assert lib.orator_gqa_decode_paged(FAKE, FAKE, FAKE, FAKE, 8, 24, FAKE, FAKE, 1, 16, 8, 128,
                                       0.1, None) == _lib.ORATOR_ERR_INVALID
    # append: k/v rows required, a positive pool size for the paged form, aligned rows
    assert lib.orator_gqa_decode_append(FAKE, None, FAKE, FAKE, FAKE, FAKE, 16, 8, 128, FAKE, 64,
                                        0.1, None) == _lib.ORATOR_ERR_INVALID
    assert lib.orator_gqa_decode_append_paged(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 8, 16, 0, FAKE,
                                              FAKE, 1, 16, 8, 128, 0.1, None) == _lib.ORATOR_ERR_INVALID
    assert lib.orator_gqa_decode_append(FAKE, FAKE + 4, FAKE, FAKE, FAKE, FAKE, 16, 8, 128, FAKE,
                                        64, 0.1, None) == _lib.ORATOR_ERR_INVALID


def test_python_wrapper_raises_gpu_error():
    from orator_amd import asr_ops
    with pytest.raises(_lib.GpuError) as e:
        asr_ops.RmsNorm(None, FAKE, FAKE, 4, 128, 1e-6)
    assert e.value.code == _lib.ORATOR_ERR_INVALID


def test_linear_and_decoder_validation():
    """asr_gemm / decoder argument checks run before any device work."""
    import ctypes as C
    lib = _lib.lib()
    # any K and any 2-byte alignment are accepted (the GPU tests run them); an odd address
    # is not a bf16 array
    assert lib.orator_linear_pre(FAKE, FAKE, None, FAKE, 4, 16, 8, 3, None) == \
        _lib.ORATOR_ERR_INVALID  # act
    assert lib.orator_linear_pre(FAKE + 1, FAKE, None, FAKE, 4, 16, 8, 0, None) == \
        _lib.ORATOR_ERR_INVALID  # alignment
    assert lib.orator_linear_pre(None, None, None, None, 0, 16, 8, 0, None) == _lib.ORATOR_OK
    cfg = _lib.DecoderConfig(1, 512, 4, 2, 64, 1024, 4096, 64, 1e-6, 1e6)
    layers = (_lib.DecoderLayer * 1)(_lib.DecoderLayer(*([FAKE] * 8)))
    h = C.c_void_p()
    assert lib.orator_decoder_create(C.byref(cfg), FAKE, FAKE, None, layers, C.byref(h)) == \
        _lib.ORATOR_ERR_UNSUPPORTED  # head_dim 64
    assert h.value is None
    cfg.head_dim, cfg.num_q_heads = 128, 3
    assert lib.orator_decoder_create(C.byref(cfg), FAKE, FAKE, None, layers, C.byref(h)) == \
        _lib.ORATOR_ERR_UNSUPPORTED  # Hq % Hkv
    cfg.num_q_heads = 4
    layers[0].o_w = None
    assert lib.orator_decoder_create(C.byref(cfg), FAKE, FAKE, None, layers, C.byref(h)) == \
        _lib.ORATOR_ERR_INVALID
    assert lib.orator_decoder_prefill_at(None, FAKE, 4, 0, None) == _lib.ORATOR_ERR_INVALID
    assert lib.orator_embed_gather(FAKE, FAKE, FAKE, 12, None) == _lib.ORATOR_ERR_INVALID


def test_decoder_rejects_context_past_decode_limit():
    import ctypes as C
    lib = _lib.lib()
    cfg = _lib.DecoderConfig(1, 512, 4, 2, 128, 1024, 4096, 131073, 1e-6, 1e6)
    layers = (_lib.DecoderLayer * 1)(_lib.DecoderLayer(*([FAKE] * 8)))
    h = C.c_void_p()
    assert lib.orator_decoder_create(C.byref(cfg), FAKE, FAKE, None, layers, C.byref(h)) == \
        _lib.ORATOR_ERR_UNSUPPORTED
    assert b"131072" in lib.orator_last_error()


def test_noalloc_decode_rejects_sizes_past_static_scratch():
    """The allocation-free decode checks its split partials against the 16 MiB static scratch
    before touching the device: B = 16, Hq = 16, Dh = 128 at 16384 keys needs ~17 MB."""
    lib = _lib.lib()
    rc = lib.orator_gqa_decode_paged_noalloc(FAKE, FAKE, FAKE, FAKE, 1024, 16, FAKE, FAKE, 16, 16,
                                             8, 128, 0.1, None)
    assert rc == _lib.ORATOR_ERR_CAPACITY
    assert b"16 MiB" in lib.orator_last_error()
    assert lib.orator_gqa_decode_paged_noalloc(FAKE, FAKE, FAKE, None, 8, 16, FAKE, FAKE, 1, 16, 8,
                                               128, 0.1, None) == _lib.ORATOR_ERR_INVALID


def test_prefill_validation():
    """orator_gqa_prefill_ex rejects, before touching the device: a paged cache past the
    16384 keys its LDS page-row table holds, a page size that is not a power of two >= 16, a
    capacity beyond max_pages * page_size, head sizes past 1024."""
    lib = _lib.lib()
    PF32 = 0

    def call(page_table, max_pages, page_size, Hq, Hkv, Dh, cap):
        return lib.orator_gqa_prefill_ex(FAKE, None, FAKE, FAKE, page_table, max_pages, page_size,
                                         FAKE, 4, Hq, Hkv, Dh, FAKE, cap, 0.1, PF32, None)

    assert call(FAKE, 1025, 16, 16, 8, 128, 16400) == _lib.ORATOR_ERR_UNSUPPORTED
    assert b"16384" in lib.orator_last_error()
    assert call(FAKE, 64, 24, 16, 8, 128, 1024) == _lib.ORATOR_ERR_INVALID
    assert call(FAKE, 64, 8, 16, 8, 128, 512) == _lib.ORATOR_ERR_INVALID
    assert call(FAKE, 16, 32, 16, 8, 128, 1024) == _lib.ORATOR_ERR_CAPACITY
    assert call(None, 0, 0, 16, 8, 2048, 1024) == _lib.ORATOR_ERR_UNSUPPORTED  # Dh > 1024
    assert call(None, 0, 0, 12, 8, 128, 1024) == _lib.ORATOR_ERR_INVALID      # Hq % Hkv
    # the generic kernel's paged form: a page size that is not a power of two, a capacity
    # beyond the table (group 8 and Dh 64 are accepted: generic shapes)
    assert call(FAKE, 64, 24, 64, 8, 128, 1024) == _lib.ORATOR_ERR_INVALID
    assert call(FAKE, 16, 32, 16, 8, 64, 1024) == _lib.ORATOR_ERR_CAPACITY
