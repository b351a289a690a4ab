"""CPU-only checks of the C-ABI library: it loads, exports every function
include/cheetah_hip.h declares, and rejects calls before initialization with
a sentence (no device work happens on this path)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cheetah_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cheetah_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from cheetah_amd import hip
    return hip.lib()


def test_header_declares_the_model_boundary():
    names = declared_functions()
    for required in ("cheetah_hip_init", "cheetah_hip_forward", "cheetah_hip_clear_cache", "cheetah_hip_clone",
                     "cheetah_hip_kv_snapshot", "cheetah_hip_restore_kv_prefix", "cheetah_hip_device_name",
                     "cheetah_hip_last_error", "cheetah_hip_gemv_q4", "cheetah_hip_attention"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    from cheetah_amd import hip
    names = declared_functions()
    assert len(names) >= 30
    for name in names:
        assert hasattr(lib, name), name
        assert name in hip.SIGNATURES, f"{name} has no ctypes signature"
    assert set(hip.SIGNATURES) == set(names)


def test_calls_before_init_fail_with_a_sentence(lib):
    from cheetah_amd import hip
    if hip._initialized:
        pytest.skip("library already initialized in this process")
    assert lib.cheetah_hip_gemv_bf16(None, 1, 1, None, None) == -1
    assert b"not initialized" in lib.cheetah_hip_last_error()
    assert lib.cheetah_hip_synchronize() == -1
    assert lib.cheetah_hip_model_create(None, 0, 0, 0, 0) is None
    assert b"not initialized" in lib.cheetah_hip_last_error()


def test_buffer_size_helpers_match_the_reference_layouts(lib):
    # q8.rs:1-25 and q4.rs:50-52 (K=4096 -> 2052-byte rows).
    assert lib.cheetah_hip_q8_buffer_bytes(4096, 4096) == 4096 * 4 + 4096 * 4096
    assert lib.cheetah_hip_q4_buffer_bytes(4096, 4096) == 4096 * 4 + 4096 * 2052
    assert lib.cheetah_hip_q4_buffer_bytes(14336, 4096) == 14336 * 4 + 14336 * 2052
    assert lib.cheetah_hip_q4_buffer_bytes(4096, 14336) == 4096 * 4 + 4096 * 7172
    assert lib.cheetah_hip_q4_buffer_bytes(3, 9) == 3 * 4 + 3 * 8
    assert lib.cheetah_hip_q8_buffer_bytes(3, 6) == 3 * 4 + 3 * 8


def test_host_wrapper_rejects_non_bf16_units():
    import numpy as np
    from cheetah_amd import configs, hip
    obj = hip.HipForward.__new__(hip.HipForward)
    obj._h = None
    obj.shape = configs.TINY_QWEN2
    with pytest.raises(hip.HipError, match="not BF16"):
        obj.set_unit("model.norm.weight", np.zeros(4, np.float32))


def test_attention_rejects_bad_geometry_before_device_work(lib):
    # Every argument error comes back as -1 with a sentence before any device
    # call (also without an initialized device): kv_heads == 0 used to reach
    # a division by zero while sizing the split grid.
    from cheetah_amd import hip
    dummy = ctypes.c_void_p(16)
    for kvh, hd, ps, q_heads, msg in [(0, 64, 64, 4, b"multiple of kv_heads"),
                                      (2, 64, 64, 3, b"multiple of kv_heads"),
                                      (2, 64, 64, 0, b"multiple of kv_heads"),
                                      (2, 0, 64, 4, b"non-zero head_dim"),
                                      (2, 64, 0, 4, b"non-zero head_dim")]:
        view = hip.KvView(16, 16, 16, ps, kvh, hd)
        assert lib.cheetah_hip_attention(dummy, ctypes.byref(view), q_heads, 1, 0, dummy) == -1
        assert msg in lib.cheetah_hip_last_error(), (kvh, hd, ps, q_heads)
    view = hip.KvView(16, 16, 16, 64, 2, 64)
    assert lib.cheetah_hip_attention(dummy, ctypes.byref(view), 4, 0, 0, dummy) == -1
    assert b"at least one query row" in lib.cheetah_hip_last_error()
