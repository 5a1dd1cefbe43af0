"""C ABI: the library loads, exports exactly what include/moe_fp8.h (the
product entry points) and include/moe_fp8_testing.h (test and measurement
instrumentation) declare,
and rejects bad arguments before touching the GPU (no compute calls here)."""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

from conftest import REPO

HEADER = REPO / "include" / "moe_fp8.h"
TESTING_HEADER = REPO / "include" / "moe_fp8_testing.h"
INSTRUMENTATION = {"moe_fill_normal_e4m3", "moe_host_fill_normal_e4m3", "moe_mfma_tiles", "moe_mfma_ceiling"}


def _declared(path) -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", path.read_text(), flags=re.S)
    return set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(moe_\w+)\s*\(", text, flags=re.M))


def declared_functions() -> set[str]:
    return _declared(HEADER) | _declared(TESTING_HEADER)


def test_instrumentation_lives_in_the_testing_header():
    assert _declared(TESTING_HEADER) == INSTRUMENTATION
    assert not (_declared(HEADER) & INSTRUMENTATION)


def test_header_declares_entry_points():
    names = declared_functions()
    assert {"moe_forward", "moe_pack_w13", "moe_pack_w2", "moe_workspace_bytes", "moe_last_error"} <= names


def test_library_exports_every_declared_symbol(lib, capi):
    names = declared_functions()
    for name in sorted(names):
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    assert names == set(capi.SIGNATURES), "ctypes prototypes must cover exactly the headers"


def test_abi_version(lib, capi):
    assert lib.moe_abi_version() == capi.ABI_VERSION
    assert f"#define MOE_ABI_VERSION {capi.ABI_VERSION}" in HEADER.read_text()


def test_packed_sizes(lib):
    assert lib.moe_packed_w13_bytes(32) == 32 * 4096 * 7168
    assert lib.moe_packed_w2_bytes(32) == 32 * 7168 * 2048
    assert lib.moe_packed_w13_bytes(0) == 0


@pytest.mark.parametrize("T,E", [(1, 32), (16, 32), (64, 32), (1000, 8), (8192, 32), (3, 1)])
def test_workspace_layout(lib, capi, T, E):
    total = lib.moe_workspace_bytes(T, E)
    off = capi.workspace_offsets(T, E)
    R = T * min(8, E)
    sizes = [T * 32, T * 32, E * 4, (E + 1) * 4, R * 4, R * 4, T * 32, R * 2048, R * 64, R * 7168 * 4,
             64 + 128 * ((T + 63) // 64)]
    assert off[0] == 0
    for b in range(capi.WS_NBUF):
        assert off[b] % 256 == 0
        end = off[b + 1] if b + 1 < capi.WS_NBUF else total
        assert end - off[b] >= sizes[b]
    assert total >= sum(sizes)


def test_workspace_invalid(lib):
    assert lib.moe_workspace_bytes(-1, 32) == 0
    assert lib.moe_workspace_bytes(16, 0) == 0
    assert lib.moe_workspace_bytes(16, 33) == 0


def _err(lib) -> str:
    return lib.moe_last_error().decode()


FAKE = ctypes.c_void_p(0x10000)  # 16-byte aligned, never dereferenced: validation fails first


def _forward(lib, T=16, E=32, ws_bytes=0, hidden=FAKE, out=FAKE, ws=FAKE):
    p = FAKE
    return lib.moe_forward(hidden, p, p, p, p, p, p, p, 2.5, 0, T, E, ws, ws_bytes, out, None)


def test_forward_rejects_bad_e_local(lib, capi):
    assert _forward(lib, E=0) == capi.MOE_ERR_INVALID_ARG
    assert "e_local" in _err(lib)
    assert _forward(lib, E=33) == capi.MOE_ERR_INVALID_ARG


def test_forward_rejects_negative_T(lib, capi):
    assert _forward(lib, T=-1) == capi.MOE_ERR_INVALID_ARG
    assert "T must be" in _err(lib)


def test_forward_rejects_T_past_max(lib, capi):
    header = (REPO / "include" / "moe_fp8.h").read_text()
    assert f"#define MOE_MAX_T {capi.MAX_T}" in header
    assert _forward(lib, T=capi.MAX_T + 1) == capi.MOE_ERR_INVALID_ARG
    assert "T must be" in _err(lib)


def test_forward_T0_is_noop(lib, capi):
    assert _forward(lib, T=0, hidden=None) == capi.MOE_OK


def test_forward_rejects_null_and_misaligned(lib, capi):
    assert _forward(lib, hidden=None) == capi.MOE_ERR_INVALID_ARG
    assert "hidden must not be null" in _err(lib)
    assert _forward(lib, out=ctypes.c_void_p(0x10004)) == capi.MOE_ERR_INVALID_ARG
    assert "16-byte aligned" in _err(lib)


def test_forward_rejects_small_workspace(lib, capi):
    need = lib.moe_workspace_bytes(16, 32)
    assert _forward(lib, ws_bytes=need - 1) == capi.MOE_ERR_WORKSPACE
    assert "workspace" in _err(lib)


def test_route_and_pack_validation(lib, capi):
    assert lib.moe_route(None, FAKE, 1.0, 0, 4, 32, FAKE, 1 << 30, None) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_route(FAKE, FAKE, 1.0, 0, 4, 40, FAKE, 1 << 30, None) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_pack_w13(None, FAKE, 32, None) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_pack_w2(FAKE, FAKE, 0, None) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_unpack_w2(FAKE, ctypes.c_void_p(0x10001), 1, None) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_fill_normal_e4m3(None, 16, 1, 1, None) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_mfma_ceiling(FAKE, FAKE, 0, 8, None) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_mfma_ceiling(FAKE, FAKE, 16, 0, None) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_mfma_ceiling(None, FAKE, 16, 8, None) == capi.MOE_ERR_INVALID_ARG


def test_capi_check_raises_runtime_error(lib, capi):
    rc = _forward(lib, E=0)
    with pytest.raises(RuntimeError, match="e_local"):
        capi.check(rc, "moe_forward")


@pytest.mark.parametrize("seed,stream,first,n", [(0, 1, 0, 4096), (0x15642003, 5, 12345, 100_003), (7, 8, 2**40, 33)])
def test_host_generator_matches_specification(ops, inputs_mod, seed, stream, first, n):
    got = ops.host_normal_e4m3(n, seed, stream, first_index=first)
    want = inputs_mod.normal_e4m3_numpy(seed, stream, n, first)
    assert np.array_equal(got, want)


def test_host_generator_threads_agree(ops):
    a = ops.host_normal_e4m3(3_000_001, 11, 3, threads=1)
    b = ops.host_normal_e4m3(3_000_001, 11, 3, threads=7)
    assert np.array_equal(a, b)


def test_noalloc_validation_before_any_gpu_work(lib, capi):
    """moe_forward_noalloc rejects sizes beyond its fixed scratch (and bad
    sizes) from the host, before touching the GPU; T == 0 is a no-op."""
    assert lib.moe_noalloc_scratch_bytes() == 32 << 20
    assert lib.moe_workspace_bytes(128, 32) <= lib.moe_noalloc_scratch_bytes()
    null = ctypes.c_void_p(0)
    rc = lib.moe_forward_noalloc(*([null] * 8), 1.0, 0, 8192, 32, null, null)
    assert rc == capi.MOE_ERR_WORKSPACE and b"scratch" in lib.moe_last_error()
    assert lib.moe_forward_noalloc(*([null] * 8), 1.0, 0, -1, 32, null, null) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_forward_noalloc(*([null] * 8), 1.0, 0, 16, 0, null, null) == capi.MOE_ERR_INVALID_ARG
    assert lib.moe_forward_noalloc(*([null] * 8), 1.0, 0, 0, 32, null, null) == capi.MOE_OK
