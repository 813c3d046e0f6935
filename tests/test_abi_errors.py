"""The error channel of the C-ABI, forced from the host: invalid shapes,
NULL handles and pointers, invalid geometries and (in this container) the
absence of a HIP device.  Every case must return an error code or, for the
reference's void entry points, NaN outputs plus tg_last_error(), never
abort.  No case reaches a kernel, so these run without a GPU; the ones that
need "no device" skip where a device is visible."""
import ctypes
import math
import os

import numpy as np
import pytest

from tinygiant_amd import _lib

NO_DEVICE = not os.path.exists("/dev/kfd")
needs_no_device = pytest.mark.skipif(not NO_DEVICE, reason="a HIP device is visible here")

TG_E_INVALID, TG_E_NODEVICE = -1, -2


@pytest.fixture(scope="module")
def lib():
    return _lib.require_lib()


def last(lib) -> str:
    return lib.tg_last_error().decode()


@needs_no_device
def test_init_without_device(lib):
    assert lib.tg_gpu_init(0) == TG_E_NODEVICE
    assert "no HIP device" in last(lib)
    assert lib.tg_device_sync() == TG_E_NODEVICE


@pytest.mark.parametrize("L,E,H,I,k,msg", [
    (0, 128, 2048, 768, 8, "n_layers"),
    (1, 128, 2000, 768, 8, "embed_dim"),
    (1, 128, 2048, 770, 8, "inter_dim"),
    (1, 130, 2048, 768, 8, "n_experts"),
    (1, 256, 2048, 768, 8, "n_experts"),
    (1, 128, 2048, 768, 0, "top_k"),
    (1, 8, 2048, 768, 12, "top_k"),
    (1, 128, 16384, 768, 8, "above"),
])
def test_arena_create_rejects_shapes(lib, L, E, H, I, k, msg):
    assert not lib.tg_arena_create(L, E, H, I, k)
    assert msg in last(lib)


@needs_no_device
def test_arena_create_without_device(lib):
    assert not lib.tg_arena_create(1, 128, 2048, 768, 8)
    assert "no HIP device" in last(lib)


def test_null_arena(lib):
    f = np.zeros(4, np.float32)
    p = f.ctypes.data
    cases = [
        lambda: lib.tg_moe_layer_q40_dev(None, 0, p, p, 1, None, None, 1e-6, None),
        lambda: lib.tg_moe_layer_q40(None, 0, p, p, 1, None, None, 1e-6),
        lambda: lib.tg_moe_stack_q40_dev(None, p, 1, 0, 1, 1e-6, None),
        lambda: lib.tg_moe_stack_q40(None, p, 1, 0, 1, 1e-6),
        lambda: lib.tg_moe_stack_q40_trace_dev(None, p, 0, 1, 1e-6, p, p, None),
        lambda: lib.tg_arena_load_layer(None, 0, p, 16),
        lambda: lib.tg_arena_load_router(None, 0, p, 4),
        lambda: lib.tg_arena_load_norm(None, 0, p, 4),
        lambda: lib.tg_arena_read_layer(None, 0, p, 16),
        lambda: lib.tg_arena_synth_layer(None, 0, 1, 0.02),
        lambda: lib.tg_arena_set_decode_path(None, 0),
        lambda: lib.tg_arena_set_batch_path(None, 0),
        lambda: lib.tg_arena_status(None),
        lambda: lib.tg_arena_expert_offset(None, 0, None, None, None, None),
    ]
    for i, c in enumerate(cases):
        assert c() == TG_E_INVALID, i
        assert "arena is NULL" in last(lib), i
    assert lib.tg_arena_expert_bytes(None) == 0 and lib.tg_arena_layer_bytes(None) == 0
    lib.tg_arena_destroy(None)  # no-op


def test_head_rejects_arguments(lib):
    W = np.zeros(8, np.float32)
    assert not lib.tg_head_create(None, W.ctypes.data, 4, 2)
    assert "tg_head_create" in last(lib)
    assert not lib.tg_head_create(W.ctypes.data, W.ctypes.data, 0, 2)
    assert "vocab 0" in last(lib)
    tok = ctypes.c_int32()
    assert lib.tg_head_forward(None, W.ctypes.data, 1e-6, None, ctypes.byref(tok)) == TG_E_INVALID
    assert "null handle" in last(lib)
    lib.tg_head_destroy(None)


def test_building_blocks_reject_arguments(lib):
    if NO_DEVICE:  # the device check comes first; its error is the one reported
        assert lib.tg_q40_quantize_q8_0_dev(None, None, 33, None) == TG_E_NODEVICE
    assert lib.tg_prof_read(None, None, None) == TG_E_INVALID


def nan_filled(a):
    return bool(np.all(np.isnan(a)))


@needs_no_device
def test_legacy_calls_fail_loudly_without_device(lib):
    """The reference's void entry points: NaN in every output element and
    the reason in tg_last_error()."""
    x = np.ones(256, np.float32)
    W = np.zeros(4 * 144, np.uint8)
    y = np.zeros(4, np.float32)
    lib.tg_matmul_q4k(W.ctypes.data, x.ctypes.data, y.ctypes.data, 4, 256)
    assert nan_filled(y) and "no HIP device" in last(lib)
    y[:] = 0
    lib.tg_matmul_q6k(W.ctypes.data, x.ctypes.data, y.ctypes.data, 4, 256)
    assert nan_filled(y)
    A = np.zeros((4, 256), np.float32)
    y[:] = 0
    lib.tg_f32_matvec(A.ctypes.data, x.ctypes.data, y.ctypes.data, 4, 256)
    assert nan_filled(y)
    out = np.zeros(256, np.float32)
    lib.tg_rms_norm(x.ctypes.data, x.ctypes.data, out.ctypes.data, 256, 1e-6)
    assert nan_filled(out)


def attention(lib, embed, n_heads, n_kv, hd, kv_len, kv_max):
    """tg_attention_decode with zero operands of the given geometry."""
    q = np.zeros(max(1, n_heads * hd * embed), np.float32)
    kv = np.zeros(max(1, n_kv * hd * embed), np.float32)
    nw = np.ones(max(1, hd), np.float32)
    cache = np.zeros(max(1, n_kv * kv_max * hd), np.float32)
    rope = np.ones(max(1, kv_max * hd // 2), np.float32)
    x = np.ones(embed, np.float32)
    out = np.zeros(embed, np.float32)
    P = lambda a: a.ctypes.data
    lib.tg_attention_decode(P(q), P(kv), P(kv), P(q), P(nw), P(nw), P(cache), P(cache), kv_len, kv_max,
                            P(rope), P(rope), P(x), P(out), embed, n_heads, n_kv, hd, kv_len)
    return out


@pytest.mark.parametrize("n_heads,n_kv,hd,kv_len,kv_max", [
    (4, 2, 64, 8, 8),      # kv_len must stay below kv_max (the new row)
    (4, 3, 64, 1, 8),      # n_heads % n_kv_heads != 0
    (2, 2, 1024, 1, 8),    # head_dim above 512
    (4, 2, 63, 1, 8),      # odd head_dim (RoPE pairs)
])
def test_attention_rejects_geometry(lib, n_heads, n_kv, hd, kv_len, kv_max):
    out = attention(lib, 64, n_heads, n_kv, hd, kv_len, kv_max)
    assert nan_filled(out)
    assert "attention geometry" in last(lib)


def test_residency_helpers_on_host_memory(lib):
    """tg_prefetch / tg_mlock keep the reference's POSIX behaviour
    (csrc/libtinygiant.c:745-766) and need no device."""
    buf = np.zeros(1 << 16, np.uint8)
    lib.tg_prefetch(buf.ctypes.data, buf.nbytes)
    ptrs = (ctypes.c_void_p * 2)(buf.ctypes.data, buf.ctypes.data + 4096)
    lens = (ctypes.c_size_t * 2)(4096, 4096)
    lib.tg_prefetch_batch(ptrs, lens, 2)
    rc = lib.tg_mlock(buf.ctypes.data, 4096)
    assert rc in (0, -1)  # mlock(2)'s own result; -1 where RLIMIT_MEMLOCK forbids it
