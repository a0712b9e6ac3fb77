"""The C ABI library: builds, loads without a GPU, exports every declared symbol,
and rejects bad arguments before touching the device."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("mis_sampler.h", "mis_attention.h", "mis_lmhead.h")]


def declared_functions() -> list[str]:
    names = []
    for h in HEADERS:
        src = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names += re.findall(r"\b(mis_\w+)\s*\(", src)
    return names


@pytest.fixture(scope="module")
def lib():
    from vllm_mps_amd import _native
    if not os.path.exists(_native.lib_path()):
        pytest.fail("libmis_sampler.so not built (run __graft_entry__.build())")
    return _native.load()


def test_header_declares_expected_api():
    names = declared_functions()
    for n in ["mis_workspace_bytes", "mis_workspace_init", "mis_sample", "mis_sample_profiled", "mis_strerror", "mis_last_hip_error",
              "mis_abi_version"]:
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    from vllm_mps_amd import _native
    out = subprocess.run(["nm", "-D", "--defined-only", _native.lib_path()], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (mis_\w+)", out))
    for n in declared_functions():
        assert n in exported, n
        assert hasattr(lib, n)
    assert set(_native.EXPORTED) == set(declared_functions())


def test_abi_version_and_strings(lib):
    from vllm_mps_amd import _native
    assert lib.mis_abi_version() == _native.ABI_VERSION == 8
    assert lib.mis_strerror(0) == b"ok"
    assert b"workspace" in lib.mis_strerror(2)
    assert b"scratch" in lib.mis_strerror(_native.ERR_SCRATCH)
    assert lib.mis_last_hip_error() == 0


def test_workspace_bytes(lib):
    for B, V in [(1, 1), (8, 32000), (256, 128256), (1024, 128256), (1, 152064)]:
        n = lib.mis_workspace_bytes(B, V, 0)
        assert n > 0 and n % 256 == 0
    assert lib.mis_workspace_bytes(256, 128256, 0) < 256 << 20


def test_argument_validation_without_gpu(lib):
    vp = ctypes.c_void_p
    fake = vp(0x1000)
    call = lambda *a: lib.mis_sample(*a)
    # bad dtype / shape / stride are rejected before any launch
    assert call(fake, 7, 1, 10, 10, fake, fake, None, None, None, fake, 1 << 20, None) == 1
    assert call(fake, 0, -1, 10, 10, fake, fake, None, None, None, fake, 1 << 20, None) == 1
    assert call(fake, 0, 1, 0, 10, fake, fake, None, None, None, fake, 1 << 20, None) == 1
    assert call(fake, 0, 1, 10, 9, fake, fake, None, None, None, fake, 1 << 20, None) == 1
    assert call(None, 0, 1, 10, 10, fake, fake, None, None, None, fake, 1 << 20, None) == 1
    assert call(fake, 0, 0, 10, 10, fake, fake, None, None, None, fake, 1 << 20, None) == 0  # empty batch
    # workspace too small / misaligned
    assert call(fake, 0, 4, 1000, 1000, fake, fake, None, None, None, fake, 16, None) == 2
    assert call(fake, 0, 4, 1000, 1000, fake, fake, None, None, None, vp(0x1008), 1 << 30, None) == 2
    # unsupported sizes
    assert call(fake, 0, 1 << 31, 10, 10, fake, fake, None, None, None, fake, 1 << 60, None) == 4
    assert call(fake, 0, 1, (1 << 30) + 1, (1 << 30) + 1, fake, fake, None, None, None, fake, 1 << 60, None) == 4
    # profiled entry needs three events
    ev = (vp * 3)(None, None, None)
    assert lib.mis_sample_profiled(fake, 0, 1, 10, 10, fake, fake, None, None, None, fake, 1 << 20, None, ev) == 1
    # the hinted entry: unknown kind bits and partial event sets (four handles) are argument errors
    lib.mis_sample_ex.argtypes = [vp, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, vp, vp, vp, vp, vp,
                                  vp, ctypes.c_size_t, vp, ctypes.c_uint, vp, vp]
    assert lib.mis_sample_ex(fake, 0, 1, 10, 10, fake, fake, None, None, None, fake, 1 << 20, None, 8, None, None) == 1
    ev4 = (vp * 4)(fake, fake, fake, None)  # the fourth event missing
    assert lib.mis_sample_ex(fake, 0, 1, 10, 10, fake, fake, None, None, None, fake, 1 << 20, None, 3, ev4, None) == 1
    assert lib.mis_sample_ex(fake, 0, 0, 10, 10, fake, fake, None, None, None, fake, 1 << 20, None, 7, None, None) == 0
    # a context pointer out of nowhere is never dereferenced before the checks above
    lib.mis_context_create.argtypes = [ctypes.POINTER(vp)]
    assert lib.mis_context_create(None) == 1
    # the allocation-free entry: the same checks, then the scratch limit, all
    # before the scratch address is looked up on a device
    na = lambda *a: lib.mis_sample_noalloc(*a)
    lib.mis_sample_noalloc.argtypes = [vp, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, vp, vp, vp,
                                       vp, vp, vp, ctypes.c_uint]
    assert na(fake, 0, 1, 10, 10, fake, fake, None, None, None, None, 8) == 1
    assert na(fake, 3, 1, 10, 10, fake, fake, None, None, None, None, 7) == 1
    assert na(fake, 0, 1, 10, 9, fake, fake, None, None, None, None, 7) == 1
    assert na(None, 0, 1, 10, 10, fake, fake, None, None, None, None, 7) == 1
    assert na(fake, 0, 0, 10, 10, fake, fake, None, None, None, None, 7) == 0
    assert na(fake, 0, 1 << 31, 10, 10, fake, fake, None, None, None, None, 7) == 4
    from vllm_mps_amd import _native
    assert lib.mis_workspace_bytes(1024, 128256, 0) > _native.SCRATCH_BYTES
    assert na(fake, 0, 1024, 128256, 128256, fake, fake, None, None, None, None, 7) == _native.ERR_SCRATCH
    for B, V, dt in [(256, 128256, 0), (1024, 128256, 1), (1024, 128256, 2), (8, 32000, 0), (1, 152064, 2)]:
        assert lib.mis_workspace_bytes(B, V, dt) <= _native.SCRATCH_BYTES, (B, V, dt)
    # the generator fill: negative or empty batches and null buffers, before any launch
    lib.mis_fill_uniforms.argtypes = [vp, vp, ctypes.c_int64, vp]
    assert lib.mis_fill_uniforms(fake, fake, -1, None) == 1
    assert lib.mis_fill_uniforms(fake, fake, 0, None) == 0
    assert lib.mis_fill_uniforms(None, fake, 4, None) == 1
    assert lib.mis_fill_uniforms(fake, None, 4, None) == 1
    assert lib.mis_fill_uniforms(fake, fake, 1 << 31, None) == 4
    # paged attention: shapes and pointers checked before any launch
    pa = lambda *a: lib.mis_paged_attention(*a)
    ok = (vp(0x1000), 64, 16, 4, 64, 2 * 16 * 4 * 64, 16 * 4 * 64, fake, fake, fake, fake, 8, fake, fake, 2, 32,
          fake, None, 0, None)
    assert pa(*ok[:14], 0, *ok[15:]) == 0                                  # empty batch
    assert pa(*ok[:3], 0, *ok[4:]) == 1                                    # n_kv_heads 0
    assert pa(*ok[:4], 96, *ok[5:]) == 4                                   # d_k 96
    assert pa(*ok[:15], 30, *ok[16:]) == 4                                 # 30 heads over 4 KV heads
    assert pa(*ok[:15], 128, *ok[16:]) == 4                                # 32 query heads per KV head
    assert pa(None, *ok[1:]) == 1
    assert pa(vp(0x1002), *ok[1:]) == 1                                    # pool not 16-byte aligned
    assert pa(*ok[:9], vp(0x1008), *ok[10:]) == 1                          # queries not 16-byte aligned
    long_ctx = (*ok[:11], 64, *ok[12:])                                    # 1024 tokens: splits need a workspace
    assert pa(*long_ctx) == 2
    # splits of 64 tokens for a small batch, 256 once the grid is full without them
    assert lib.mis_paged_attention_workspace_bytes(2, 32, 4, 64, 64) == 256
    assert lib.mis_paged_attention_workspace_bytes(2, 32, 4, 64, 1024) == 2 * 32 * 16 * (64 + 2) * 4
    assert lib.mis_paged_attention_workspace_bytes(256, 32, 8, 128, 2048) == 256 * 32 * 8 * (128 + 2) * 4
    assert lib.mis_gather_kv(fake, 64, 16, 4, 64, 4096, 2048, fake, 8, fake, 2, -1, fake, fake, None) == 1
    assert lib.mis_gather_kv(fake, 64, 16, 4, 64, 4096, 2048, fake, 8, fake, -2, 16, fake, fake, None) == 1
    # fused lm_head + greedy: shapes, dtype, alignment and workspace checked before any launch
    lh = lambda *a: lib.mis_lm_head_greedy(*a)
    okh = (fake, 4096, fake, 4096, 4, 4096, 32000, 2, fake, fake, 1 << 20, None)
    assert lh(*okh[:4], 0, *okh[5:]) == 0                                  # empty batch
    assert lh(*okh[:4], -1, *okh[5:]) == 1
    assert lh(*okh[:7], 0, *okh[8:]) == 4                                  # fp32 weights
    assert lh(*okh[:3], 4000, *okh[4:]) == 1                               # weight rows shorter than H
    assert lh(fake, 4000, fake, 4000, 4, 4000, 32000, 2, fake, fake, 1 << 20, None) == 4   # H not a multiple of 64
    assert lh(vp(0x1008), *okh[1:]) == 1                                   # hidden not 16-byte aligned
    assert lh(*okh[:9], None, 0, None) == 2                                # no workspace
    assert lh(*okh[:10], 100, None) == 2                                   # too small
    assert lib.mis_lm_head_greedy_workspace_bytes(4, 32000) == ((250 * 4 * 8 + 255) // 256) * 256


def test_product_path_fails_loudly_without_library(tmp_path):
    code = ("import os; os.environ['MIS_SAMPLER_LIB']='/nonexistent/lib.so';"
            "from vllm_mps_amd import _native\n"
            "try:\n    _native.load()\nexcept _native.MisError as e:\n    print('raised', e)\n")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=ROOT)
    assert "raised" in out.stdout and "no CPU fallback" in out.stdout


def test_sampler_rejects_cpu_tensors():
    import torch
    from vllm_mps_amd import Sampler, SamplingParams, _native
    with pytest.raises(_native.MisError):
        Sampler().sample(torch.zeros(10), SamplingParams())
