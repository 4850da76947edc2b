"""CPU checks of the C-ABI boundary: libsparkq.so loads, exports every entry
point include/sparkq.h declares, and rejects bad arguments with the right
status before touching a device (no compute calls without a GPU)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "sparkq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sparkq_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = _declared()
    for required in ("sparkq_w4a16_linear", "sparkq_w4a16_dequantize", "sparkq_w4_quantize",
                     "sparkq_a8_quantize_per_token", "sparkq_int8_matmul_i32",
                     "sparkq_w8a8_linear", "sparkq_int8kv_sdpa_decode", "sparkq_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from sparkq import _lib

    handle = ctypes.CDLL(_lib.library_path())
    missing = [n for n in _declared() if not hasattr(handle, n)]
    assert not missing, missing
    # the Python binding covers the whole header too
    assert set(_declared()) <= set(_lib.SIGNATURES)


def test_abi_version_and_workspace_queries():
    from sparkq import _lib

    lib = _lib.lib()
    assert lib.sparkq_abi_version() == 1
    assert lib.sparkq_w4a16_workspace_bytes(0, 1, 1, 64) == 0
    # the M <= 4 decode GEMV keeps whole rows in one workgroup: no workspace
    assert lib.sparkq_w4a16_workspace_bytes(1, 2560, 9728, 64) == 0
    assert lib.sparkq_w4a16_workspace_bytes(4, 19456, 2560, 64) == 0
    # wider decode batches split K across workgroups
    assert lib.sparkq_w4a16_workspace_bytes(8, 2560, 9728, 64) > 0
    assert lib.sparkq_w4a16_workspace_bytes(16, 2560, 9728, 64) > 0
    # prefill: the group-sum prologue buffer [K/G][M] fp32
    assert lib.sparkq_w4a16_workspace_bytes(2048, 19456, 2560, 64) >= 2048 * 40 * 4
    assert lib.sparkq_w8a8_workspace_bytes(16, 2560, 9728) >= 16 * 9728 + 16 * 4
    assert lib.sparkq_int8kv_sdpa_workspace_bytes(1, 32, 1, 128) == 0


P = ctypes.c_void_p


def _rc(name, *args):
    from sparkq import _lib

    rc = getattr(_lib.lib(), name)(*args)
    return rc, _lib.lib().sparkq_last_error().decode()


def test_invalid_arguments_rejected_without_a_device():
    dummy = P(4096)
    # null pointer
    rc, msg = _rc("sparkq_w4a16_linear", None, dummy, dummy, dummy, dummy, 1, 64, 64, 64, 4,
                  2, 2, None, 0, None)
    assert rc == -1 and "null" in msg
    # bits other than 4 is unsupported
    rc, msg = _rc("sparkq_w4a16_linear", dummy, dummy, dummy, dummy, dummy, 1, 64, 64, 64, 8,
                  2, 2, None, 0, None)
    assert rc == -2 and "bits" in msg
    # bad group size
    rc, msg = _rc("sparkq_w4a16_linear", dummy, dummy, dummy, dummy, dummy, 1, 64, 64, 48, 4,
                  2, 2, None, 0, None)
    assert rc == -1 and "group_size" in msg
    # K not a multiple of 32 for the int8 path (X/src/spark_w8a8.cpp:58-60)
    rc, msg = _rc("sparkq_int8_matmul_i32", dummy, dummy, dummy, 1, 64, 48, None, 0, None)
    assert rc == -1 and "multiple of 32" in msg
    rc, msg = _rc("sparkq_int8_matmul_i32", dummy, dummy, dummy, 1, 64, 131072, None, 0, None)
    assert rc == -1 and "131040" in msg
    # fp32 activations are not a W4A16 input
    rc, msg = _rc("sparkq_w4a16_linear", dummy, dummy, dummy, dummy, dummy, 1, 64, 64, 64, 4,
                  0, 0, None, 0, None)
    assert rc == -2
    # attention: heads not divisible by KV heads
    st = (ctypes.c_int64 * 12)(*([128] * 12))
    rc, msg = _rc("sparkq_int8kv_sdpa_decode", dummy, dummy, dummy, None, dummy, dummy, None,
                  dummy, 1, 6, 4, 16, 128, 32, 0, 2, 2, ctypes.c_float(0.1), st, None, 0, None)
    assert rc == -1 and "divisible" in msg
    # attention: unsupported head dim
    rc, msg = _rc("sparkq_int8kv_sdpa_decode", dummy, dummy, dummy, None, dummy, dummy, None,
                  dummy, 1, 8, 8, 16, 96, 32, 0, 2, 2, ctypes.c_float(0.1), st, None, 0, None)
    assert rc == -2 and "head dim" in msg
    # attention: non-finite scale
    rc, msg = _rc("sparkq_int8kv_sdpa_decode", dummy, dummy, dummy, None, dummy, dummy, None,
                  dummy, 1, 8, 8, 16, 128, 32, 0, 2, 2, ctypes.c_float(float("inf")), st,
                  None, 0, None)
    assert rc == -1 and "finite" in msg
    # W8A16: fp32 activations, more than 4 rows, K not a multiple of 16
    rc, msg = _rc("sparkq_w8a16_linear", dummy, dummy, dummy, dummy, 1, 64, 64, 0, 0, None)
    assert rc == -1 and "bfloat16 or float16" in msg
    rc, msg = _rc("sparkq_w8a16_linear", dummy, dummy, dummy, dummy, 5, 64, 64, 2, 2, None)
    assert rc == -2 and "4 activation rows" in msg
    rc, msg = _rc("sparkq_w8a16_linear", dummy, dummy, dummy, dummy, 1, 64, 40, 2, 2, None)
    assert rc == -2 and "multiple of 16" in msg


def test_layer_entry_points_validate_without_a_device():
    dummy = P(4096)
    f = ctypes.c_float
    ffn = lambda m, k, i, g, dt, eps=1e-6: _rc(  # noqa: E731
        "sparkq_ffn", dummy, dummy, dummy, f(eps), *([dummy] * 9), dummy, m, k, i, g, dt,
        None, 0, None)
    rc, msg = ffn(1, 2560, 9728, 48, 2)
    assert rc == -1 and "group_size" in msg
    rc, msg = ffn(1, 2560, 9700, 64, 2)
    assert rc == -2 and "multiples of 64" in msg
    rc, msg = ffn(1, 2560, 9728, 64, 0)
    assert rc == -2 and "bfloat16 or float16" in msg
    rc, msg = ffn(1, 2560, 9728, 64, 2, eps=float("nan"))
    assert rc == -1 and "eps" in msg
    from sparkq import _lib

    lib = _lib.lib()
    # workspace: counters of the projections, hidden, normed, act, gate, up
    assert lib.sparkq_ffn_workspace_bytes(1, 2560, 9728, 64) >= 2 * 2560 * 2 + 3 * 9728 * 2
    assert lib.sparkq_ffn_workspace_bytes(0, 2560, 9728, 64) == 0
    assert lib.sparkq_qkv_rope_workspace_bytes(2560, 32, 8, 128, 64) >= 3584 * 2

    def qkv(q_size=4096, kv_size=1024, nh=32, nkv=8, hd=128, rd=128, base=10000.0, g=64, bits=4,
            hidden=2560, off=0):
        return _rc("sparkq_qkv_rope", dummy, dummy, dummy, dummy, dummy, dummy, dummy, hidden,
                   q_size, kv_size, nh, nkv, hd, rd, f(base), off, g, bits, 2, None, 0, None)

    # the reference's checks and messages (X/src/spark_qkv_rope.cpp:29-81)
    rc, msg = qkv(nkv=5)
    assert rc == -1 and "Invalid head counts" in msg
    rc, msg = qkv(q_size=4000)
    assert rc == -1 and "Invalid head counts" in msg
    rc, msg = qkv(rd=7)
    assert rc == -1 and "rope_dims must be positive, even" in msg
    rc, msg = qkv(rd=256)
    assert rc == -1 and "rope_dims" in msg
    rc, msg = qkv(base=-1.0)
    assert rc == -1 and "rope_base" in msg
    rc, msg = qkv(g=16)
    assert rc == -1 and "group_size must be 32, 64, or 128" in msg
    rc, msg = qkv(bits=7)
    assert rc == -1 and "bits must be 1, 2, 3, 4, 5, 6, or 8" in msg
    rc, msg = qkv(bits=8)
    assert rc == -2 and "bits=4" in msg
    rc, msg = qkv(hidden=2500)
    assert rc == -1 and "metadata shapes" in msg
    rc, msg = _rc("sparkq_rope", dummy, dummy, 6, 4, 128, 128, 0, f(10000.0), f(1.0), 0, 2, None)
    assert rc == -1 and "multiple of L" in msg
    rc, msg = _rc("sparkq_rope", dummy, dummy, 8, 4, 128, 130, 0, f(10000.0), f(1.0), 0, 2, None)
    assert rc == -1 and "dims" in msg
    rc, msg = _rc("sparkq_rms_norm", dummy, None, dummy, f(1e-6), None, dummy, 1, 64, 0, None)
    assert rc == -2 and "bfloat16 or float16" in msg


def test_status_maps_to_reference_exceptions():
    from sparkq import _lib

    with pytest.raises(ValueError, match="null"):
        _lib.call("sparkq_a8_quantize_per_token", None, None, None, 1, 32, 2, None)


def test_ranges_beyond_one_buffer_descriptor_are_unsupported():
    """Kernels address a tensor (or one sequence's KV slice) with 32-bit
    buffer offsets and use offset 2^31 for lanes with nothing to read, so any
    such range above 2 GiB must be refused before a launch, not wrapped."""
    dummy = P(4096)
    f = ctypes.c_float
    # W4: a 2^20 x 2^13 weight is 4 GiB of packed codes
    rc, msg = _rc("sparkq_w4a16_linear", dummy, dummy, dummy, dummy, dummy, 1, 1 << 20,
                  1 << 13, 64, 4, 2, 2, None, 0, None)
    assert rc == -2 and "2 GiB" in msg
    # W8: an int8 head of 262144 x 16384 (4 GiB)
    rc, msg = _rc("sparkq_w8a16_linear", dummy, dummy, dummy, dummy, 1, 262144, 16384, 2, 2,
                  None)
    assert rc == -2 and "2 GiB" in msg
    rc, msg = _rc("sparkq_int8_matmul_i32", dummy, dummy, dummy, 1, 262144, 16384, None, 0,
                  None)
    assert rc == -2 and "2 GiB" in msg
    rc, msg = _rc("sparkq_w8a8_linear", dummy, dummy, dummy, None, 0, dummy, 1, 262144, 16384,
                  2, 2, dummy, 0, None)
    assert rc == -2 and "2 GiB" in msg
    # exactly 2 GiB is still addressable: 131072 x 16384 int8
    rc, msg = _rc("sparkq_w8a16_linear", dummy, dummy, dummy, dummy, 1, 131072, 16384, 2, 2,
                  None)
    assert "2 GiB" not in msg
    # attention: a token stride of 64 KiB over 2^16 tokens is a 4 GiB slice
    big = (ctypes.c_int64 * 12)(0, 0, 65536, 0, 0, 1, 0, 0, 65536, 0, 0, 1)
    rc, msg = _rc("sparkq_int8kv_sdpa_decode", dummy, dummy, dummy, None, dummy, dummy, None,
                  dummy, 1, 8, 8, 65536, 128, 32, 0, 2, 2, f(0.1), big, None, 0, None)
    assert rc == -2 and "32-bit offsets" in msg
    rc, msg = _rc("sparkq_int8kv_sdpa_prefill", dummy, dummy, dummy, dummy, dummy, dummy, 1, 8,
                  8, 2, 65536, 128, 1, 2, 2, f(0.1), big, None)
    assert rc == -2 and "32-bit offsets" in msg
    # a broadcast (zero) token stride would make the range empty: refused
    zero = (ctypes.c_int64 * 12)(0, 0, 0, 0, 0, 1, 0, 0, 128, 0, 0, 1)
    rc, msg = _rc("sparkq_int8kv_sdpa_decode", dummy, dummy, dummy, None, dummy, dummy, None,
                  dummy, 1, 8, 8, 16, 128, 32, 0, 2, 2, f(0.1), zero, None, 0, None)
    assert rc == -1 and "token strides must be positive" in msg
    rc, msg = _rc("sparkq_int8kv_sdpa_prefill", dummy, dummy, dummy, dummy, dummy, dummy, 1, 8,
                  8, 2, 16, 128, 1, 2, 2, f(0.1), zero, None)
    assert rc == -1 and "token strides must be positive" in msg
    aff = (ctypes.c_int64 * 12)(0, 0, 0, 0, 0, 4, 0, 0, 32, 0, 0, 4)
    rc, msg = _rc("sparkq_int8kv_sdpa_prefill_affine", dummy, dummy, dummy, dummy, dummy, dummy,
                  dummy, dummy, 1, 8, 8, 2, 16, 128, 32, 1, 2, 2, f(0.1), aff, None, 0, None)
    assert rc == -1 and "token strides must be positive" in msg


def test_noalloc_decode_refuses_oversized_scratch_without_a_device():
    """The allocation-free decode keeps a fixed 8 MiB scratch per GPU: a
    split decode that needs more (here 256 query heads of 256 dims) is
    refused before any device call; 64 heads at D=256 fit."""
    from sparkq import _lib

    dummy = P(4096)
    st = (ctypes.c_int64 * 12)(0, 0, 256, 0, 0, 1, 0, 0, 256, 0, 0, 1)
    need = _lib.lib().sparkq_int8kv_sdpa_workspace_bytes(1, 256, 32768, 256)
    assert need > 8 << 20
    rc, msg = _rc("sparkq_int8kv_sdpa_decode_noalloc", dummy, dummy, dummy, None, dummy, dummy,
                  None, dummy, 1, 256, 32, 32768, 256, 32, 0, 2, 2, ctypes.c_float(0.1), st, None)
    assert rc == -2 and "scratch" in msg
    for b in (1, 2, 3, 8, 64):
        assert _lib.lib().sparkq_int8kv_sdpa_workspace_bytes(b, 64, 32768, 256) <= 8 << 20
