"""CPU checks of the C-ABI boundary: the four drop-in libraries load, export
every symbol include/dsv4_kernels.h declares under the reference's file
names, and return the reference's error codes from host-side validation
(which runs before any HIP call, so no GPU is needed)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from tests.conftest import PKG, REPO

HEADER = os.path.join(REPO, "include", "dsv4_kernels.h")

LIBS = {
    "mxfp4-routed/libmxfp4_grouped_gemv.so": [
        "mxfp4_grouped_gemv_topk", "mxfp4_grouped_workspace_bytes",
        "mxfp4_moe_route_sigmoid_topk", "mxfp4_moe_workspace_bytes", "mxfp4_moe_grouped_gemv",
        "mxfp4_moe_build_routing", "mxfp4_moe_swiglu", "mxfp4_moe_down", "mxfp4_moe_layer",
        "mxfp4_moe_prefill_workspace_bytes", "mxfp4_moe_prefill", "mxfp4_moe_prefill_dequant_bf16",
        "mxfp4_moe_route_topk", "mxfp4_moe_router_logits", "mxfp4_moe_dispatch_workspace_bytes",
        "mxfp4_moe_routed_dispatch", "mxfp4_moe_grouped_gemv_noalloc", "mxfp4_moe_gate_swiglu"],
    "mxfp4-dense/libmxfp4_gemv.so": ["mxfp4_gemv_m1", "mxfp4_dequant_bf16"],
    "fp8-dense/libfp8_e4m3_gemv.so": ["fp8_e4m3_gemv_m1", "fp8_e4m3_gemv", "fp8_e4m3_gemv_grouped",
                                      "fp8_e4m3_gemv_multi", "fp8_e4m3_gemv_f32s",
                                      "fp8_e4m3_swiglu_gemv", "fp8_e4m3_rmsnorm_gemv", "fp8_e4m3_dequant_bf16"],
    "rmsnorm-fuse/librmsnorm_fuse.so": ["rmsnorm_fuse_fwd", "rmsnorm_fuse_residual_add"],
}

# Symbols the reference engine resolves with dlsym / extern / weak reference
# (kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4.cu:149-154, routed.cu:46-54, head.cu:302-312).
REFERENCE_SYMBOLS = ["fp8_e4m3_gemv_m1", "mxfp4_grouped_gemv_topk", "mxfp4_grouped_workspace_bytes",
                     "rmsnorm_fuse_fwd", "rmsnorm_fuse_residual_add", "mxfp4_gemv_m1"]


def _lib(rel):
    path = os.path.join(PKG, "kernel", rel)
    if not os.path.exists(path):
        pytest.fail(f"{path} missing: run __graft_entry__.build() first")
    return ctypes.CDLL(path)


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+(\w+)\s*\(", text, flags=re.M)))


STORE_HEADER = os.path.join(REPO, "include", "dsv4_expert_store.h")
STORE_LIB = "expert-store/libdsv4_expert_store.so"


def test_expert_store_header_matches_exports():
    text = re.sub(r"/\*.*?\*/", "", open(STORE_HEADER).read(), flags=re.S)
    declared = sorted(set(re.findall(r"^\s*(?:int|dsv4_store\s*\*)\s*(\w+)\s*\(", text, flags=re.M)))
    assert declared == ["dsv4_store_close", "dsv4_store_count", "dsv4_store_load_experts",
                        "dsv4_store_load_tensor", "dsv4_store_open", "dsv4_store_read",
                        "dsv4_store_tensor_info"]
    lib = _lib(STORE_LIB)
    for sym in declared:
        assert hasattr(lib, sym), f"{STORE_LIB} does not export {sym}"


def test_header_declares_exactly_the_exported_set():
    declared = _declared()
    exported = sorted(s for syms in LIBS.values() for s in syms)
    assert declared == exported
    assert set(REFERENCE_SYMBOLS) <= set(declared)


@pytest.mark.parametrize("rel", sorted(LIBS))
def test_library_exports_symbols(rel):
    lib = _lib(rel)
    for sym in LIBS[rel]:
        assert hasattr(lib, sym), f"{rel} does not export {sym}"
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(PKG, "kernel", rel)],
                         capture_output=True, text=True, check=True).stdout
    for sym in LIBS[rel]:
        assert re.search(rf"\bT {sym}$", out, flags=re.M), f"{sym} not a defined text symbol"


def test_header_compiles_as_c():
    src = f'#include "{HEADER}"\nint main(void) {{ return 0; }}\n'
    r = subprocess.run(["gcc", "-x", "c", "-std=c99", "-fsyntax-only", "-I/opt/rocm/include",
                        "-D__HIP_PLATFORM_AMD__", "-"], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


N = None  # null device pointer: validation returns before any device access


def test_grouped_validation_codes():
    lib = _lib("mxfp4-routed/libmxfp4_grouped_gemv.so")
    f = lib.mxfp4_grouped_gemv_topk
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_int] * 4 + [ctypes.c_void_p] * 3

    def call(K, H, O, n):
        return f(N, N, N, N, N, N, N, N, K, H, O, n, N, N, N)

    assert call(4095, 2048, 4096, 8) == -1
    assert call(4096, 2047, 4096, 8) == -2
    assert call(4128, 2048, 4096, 8) == -3
    assert call(4096, 4128, 4096, 8) == -3
    assert call(4096, 2048, 4096, 0) == -4
    assert call(4096, 2048, 4096, 257) == -4
    assert call(4096, 2048, 0, 8) == -6
    ws = lib.mxfp4_grouped_workspace_bytes
    ws.restype = ctypes.c_size_t
    ws.argtypes = [ctypes.c_int] * 3
    assert ws(6, 2048, 4096) == 6 * 2048 * 2 + 4096 * 4  # reference formula
    assert ws(8, 2048, 4096) == 49152


def test_moe_validation_codes():
    lib = _lib("mxfp4-routed/libmxfp4_grouped_gemv.so")
    f = lib.mxfp4_moe_grouped_gemv
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 9 + [ctypes.c_int] * 6 + [ctypes.c_void_p] * 3

    def call(T, k, E, K, H, O):
        return f(N, N, N, N, N, N, N, N, N, T, k, E, K, H, O, N, N, N)

    assert call(1, 8, 256, 4095, 2048, 4096) == -1
    assert call(1, 8, 256, 4096, 2047, 4096) == -2
    assert call(1, 8, 256, 8192, 2048, 4096) == -3
    assert call(0, 8, 256, 4096, 2048, 4096) == -4
    assert call(65, 8, 256, 4096, 2048, 4096) == -4
    assert call(1, 17, 256, 4096, 2048, 4096) == -4
    assert call(1, 8, 1025, 4096, 2048, 4096) == -4
    r = lib.mxfp4_moe_route_sigmoid_topk
    r.restype = ctypes.c_int
    r.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 3
    assert r(N, 0, 256, 8, N, N, N) == -1
    assert r(N, 1, 4, 8, N, N, N) == -1
    assert r(N, 1, 256, 17, N, N, N) == -1
    wb = lib.mxfp4_moe_workspace_bytes
    wb.restype = ctypes.c_size_t
    wb.argtypes = [ctypes.c_int] * 4
    assert wb(16, 8, 256, 2048) >= 16 * 8 * 2048 * 2
    assert wb(0, 8, 256, 2048) == 0


def test_noalloc_validation_codes():
    """The no-allocation entry validates like mxfp4_moe_grouped_gemv and rejects
    shapes whose tables and intermediate exceed its 4 MiB device array, all
    before any HIP call."""
    lib = _lib("mxfp4-routed/libmxfp4_grouped_gemv.so")
    f = lib.mxfp4_moe_grouped_gemv_noalloc
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 9 + [ctypes.c_int] * 6 + [ctypes.c_void_p] * 2

    def call(T, k, E, K, H, O):
        return f(N, N, N, N, N, N, N, N, N, T, k, E, K, H, O, N, N)

    assert call(1, 8, 256, 4095, 2048, 4096) == -1
    assert call(1, 8, 256, 4096, 2047, 4096) == -2
    assert call(65, 8, 256, 4096, 2048, 4096) == -4
    assert call(64, 16, 256, 4096, 4096, 4096) == -8     # 1024 rows x 8 KiB of intermediate
    assert call(64, 16, 256, 4096, 2048, 4096) == -8     # 4 MiB + tables
    wb = lib.mxfp4_moe_workspace_bytes
    wb.restype = ctypes.c_size_t
    wb.argtypes = [ctypes.c_int] * 4
    assert wb(16, 8, 256, 2048) <= 4 << 20                 # the configuration's T <= 16 fits


def test_moe_extensions_reject_null_operands():
    """Every routed-MoE extension returns -10 when a required pointer is null,
    after the shape checks and before any HIP call (one pointer null at a
    time, the others set to an address that is never dereferenced); the
    optional ids_out / weights_out of the layer entries are not required."""
    lib = _lib("mxfp4-routed/libmxfp4_grouped_gemv.so")
    P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    D = ctypes.c_void_p(1 << 20)   # stand-in address; validation never reads it

    def each_null(fn, argtypes, build, n_ptr):
        fn.restype = I
        fn.argtypes = argtypes
        for i in range(n_ptr):
            ptrs = [D] * n_ptr
            ptrs[i] = N
            assert fn(*build(ptrs)) == -10, f"{fn.__name__}: pointer {i}"

    shape = (1, 8, 256, 4096, 2048, 4096)       # T, topk, n_experts, K_in, hidden, out_dim
    each_null(lib.mxfp4_moe_grouped_gemv, [P] * 9 + [I] * 6 + [P] * 3,
              lambda p: p[:9] + list(shape) + p[9:] + [N], 11)
    each_null(lib.mxfp4_moe_grouped_gemv_noalloc, [P] * 9 + [I] * 6 + [P] * 2,
              lambda p: p[:9] + list(shape) + p[9:] + [N], 10)
    # x, logits, W1..S2 (8), out, workspace; ids_out / weights_out stay null
    each_null(lib.mxfp4_moe_layer, [P] * 8 + [I] * 6 + [P] * 5,
              lambda p: p[:8] + list(shape) + [p[8], N, N, p[9], N], 10)
    each_null(lib.mxfp4_moe_gate_swiglu, [P] * 6 + [I] * 5 + [P] * 4,
              lambda p: p[:6] + list(shape[:5]) + [N, N, p[6], N], 7)
    each_null(lib.mxfp4_moe_build_routing, [P, P] + [I] * 4 + [P, P],
              lambda p: [p[0], p[1], 1, 8, 256, 2048, p[2], N], 3)
    each_null(lib.mxfp4_moe_swiglu, [P] * 5 + [I] * 5 + [P, P],
              lambda p: p[:5] + list(shape[:5]) + [p[5], N], 6)
    each_null(lib.mxfp4_moe_down, [P, P] + [I] * 5 + [P, P, P],
              lambda p: [p[0], p[1], 1, 8, 256, 2048, 4096, p[2], p[3], N], 4)
    each_null(lib.mxfp4_moe_route_sigmoid_topk, [P, I, I, I, P, P, P],
              lambda p: [p[0], 1, 256, 8, p[1], p[2], N], 3)
    each_null(lib.mxfp4_moe_route_topk, [P, I, I, I, I, F, P, P, P],
              lambda p: [p[0], 1, 256, 6, 1, 1.5, p[1], p[2], N], 3)
    # x, W_gate, W1..S2 (6), out, workspace; ids_out / weights_out stay null
    each_null(lib.mxfp4_moe_routed_dispatch, [P] * 8 + [I] * 6 + [F] + [P] * 5,
              lambda p: p[:8] + [1, 6, 256, 4096, 2048, 4096, 1.5, p[8], N, N, p[9], N], 10)


def test_router_and_dispatch_validation_codes():
    lib = _lib("mxfp4-routed/libmxfp4_grouped_gemv.so")
    P, I = ctypes.c_void_p, ctypes.c_int
    rt = lib.mxfp4_moe_route_topk
    rt.restype = I
    rt.argtypes = [P, I, I, I, I, ctypes.c_float, P, P, P]
    assert rt(N, 1, 256, 6, 2, 1.5, N, N, N) == -1      # unknown score mode
    assert rt(N, 1, 256, 6, -1, 1.5, N, N, N) == -1
    assert rt(N, 0, 256, 6, 1, 1.5, N, N, N) == -1      # T < 1
    assert rt(N, 1, 4, 6, 1, 1.5, N, N, N) == -1        # topk > n_experts
    rl = lib.mxfp4_moe_router_logits
    rl.restype = I
    rl.argtypes = [P, P, I, I, I, P, P]
    assert rl(N, N, 0, 256, 4096, N, N) == -1            # T < 1
    assert rl(N, N, 65, 256, 4096, N, N) == -1           # T > 64
    assert rl(N, N, 1, 1025, 4096, N, N) == -1           # n_experts > 1024
    assert rl(N, N, 1, 256, 4100, N, N) == -1            # K % 8
    assert rl(N, N, 1, 256, 8200, N, N) == -1            # K > 8192
    assert rl(ctypes.c_void_p(8), N, 1, 256, 4096, N, N) == -3  # unaligned x
    ws = lib.mxfp4_moe_dispatch_workspace_bytes
    ws.restype = ctypes.c_size_t
    ws.argtypes = [I] * 4
    wm = lib.mxfp4_moe_workspace_bytes
    wm.restype = ctypes.c_size_t
    wm.argtypes = [I] * 4
    assert ws(1, 6, 256, 2048) >= wm(1, 6, 256, 2048) + 256 * 4
    assert ws(0, 6, 256, 2048) == 0
    d = lib.mxfp4_moe_routed_dispatch
    d.restype = I
    d.argtypes = [P] * 8 + [I] * 6 + [ctypes.c_float] + [P] * 5

    def call(T, k, E, K, H, O):
        return d(*([N] * 8), T, k, E, K, H, O, 1.5, N, N, N, N, N)

    assert call(1, 6, 256, 4095, 2048, 4096) == -1
    assert call(1, 6, 256, 4096, 2047, 4096) == -2
    assert call(1, 6, 256, 8192, 2048, 4096) == -3
    assert call(1, 300, 256, 4096, 2048, 4096) == -4
    assert call(1, 8, 4, 4096, 2048, 4096) == -4          # topk > n_experts
    assert call(1, 6, 256, 4096, 2048, 4096) == -10       # null operands
    pd = lib.mxfp4_moe_prefill_dequant_bf16
    pd.restype = I
    pd.argtypes = [P, P, I, I, P, P]
    assert pd(N, N, 100, 4, N, N) == -1
    assert pd(N, N, 128, 4, N, N) == -3


def test_prefill_validation_codes():
    lib = _lib("mxfp4-routed/libmxfp4_grouped_gemv.so")
    P = ctypes.c_void_p
    fn = lib.mxfp4_moe_prefill
    fn.restype = ctypes.c_int
    fn.argtypes = [P] * 9 + [ctypes.c_int] * 6 + [P] * 3
    ws = lib.mxfp4_moe_prefill_workspace_bytes
    ws.restype = ctypes.c_size_t
    ws.argtypes = [ctypes.c_int] * 5

    def call(T, topk, E, K, H, O):
        return fn(*([None] * 9), T, topk, E, K, H, O, None, None, None)

    assert call(512, 8, 256, 4000, 2048, 4096) == -1      # K_in % 128
    assert call(512, 8, 256, 16384, 2048, 4096) == -1     # K_in > 8192
    assert call(512, 8, 256, 4096, 2000, 4096) == -2      # hidden % 128
    assert call(512, 8, 256, 4096, 2048, 4000) == -3      # out_dim % 64
    assert call(0, 8, 256, 4096, 2048, 4096) == -4        # T < 1
    assert call(512, 17, 256, 4096, 2048, 4096) == -4     # topk > 16
    assert call(512, 8, 2048, 4096, 2048, 4096) == -4     # n_experts > 1024
    assert call(512, 8, 256, 4096, 2048, 4096) == -3      # null operands
    assert ws(0, 8, 256, 2048, 4096) == 0
    big = ws(512, 8, 256, 2048, 4096)
    # M [P, H] bf16 + Y [P, O] fp32 dominate
    assert big >= 4096 * 2048 * 2 + 4096 * 4096 * 4


def test_dense_validation_codes():
    lib = _lib("mxfp4-dense/libmxfp4_gemv.so")
    f = lib.mxfp4_gemv_m1
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 2 + [ctypes.c_int64] * 2 + [ctypes.c_void_p] * 2
    assert f(N, N, N, 4095, 2048, 2048, 128, N, N) == -1
    assert f(N, N, N, 8224, 2048, 4112, 257, N, N) == -2
    assert f(N, N, N, 4096, 0, 2048, 128, N, N) == -3
    d = lib.mxfp4_dequant_bf16
    d.restype = ctypes.c_int
    d.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int] * 2 + [ctypes.c_int64] * 2 + [ctypes.c_void_p] * 2
    assert d(N, N, 100, 4, 50, 4, N, N) == -1


def test_fp8_validation_codes():
    lib = _lib("fp8-dense/libfp8_e4m3_gemv.so")
    f = lib.fp8_e4m3_gemv_m1
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 2 + [ctypes.c_int64] * 2 + [ctypes.c_void_p] * 2
    assert f(N, N, N, 4000, 1536, 4000, 32, N, N) == -1
    assert f(N, N, N, 16512, 1536, 16512, 129, N, N) == -3
    assert f(N, N, N, 4096, 0, 4096, 32, N, N) == -4
    g = lib.fp8_e4m3_gemv
    g.restype = ctypes.c_int
    P, I, L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    g.argtypes = [P, L, P, P, I, I, I, L, L, P, L, P]
    assert g(N, 4096, N, N, 4096, 1536, 0, 4096, 32, N, 1536, N) == -5
    assert g(N, 4096, N, N, 4096, 1536, 17, 4096, 32, N, 1536, N) == -5
    assert g(N, 4096, N, N, 4000, 1536, 2, 4096, 32, N, 1536, N) == -1
    gr = lib.fp8_e4m3_gemv_grouped
    gr.restype = I
    gr.argtypes = [P, L, L, P, P, I, I, I, I, L, L, P, L, L, P]
    assert gr(N, 32768, 4096, N, N, 0, 4096, 1024, 1, 4096, 32, N, 8192, 1024, N) == -6
    assert gr(N, 32768, 4096, N, N, 8, 4096, 1024, 17, 4096, 32, N, 8192, 1024, N) == -5
    assert gr(N, 32768, 4096, N, N, 8, 4000, 1024, 1, 4096, 32, N, 8192, 1024, N) == -1
    sw = lib.fp8_e4m3_swiglu_gemv
    sw.restype = I
    sw.argtypes = [P, L, P, P, P, P, I, I, I, L, L, ctypes.c_float, I, P, L, P]
    assert sw(N, 4096, N, N, N, N, 4096, 2048, 0, 4096, 32, 10.0, 1, N, 2048, N) == -5
    assert sw(N, 4096, N, N, N, N, 4000, 2048, 1, 4096, 32, 10.0, 1, N, 2048, N) == -1
    # K = 512 is a valid GEMV shape that the fused kernel does not take
    assert sw(N, 512, N, N, N, N, 512, 2048, 1, 512, 4, 10.0, 1, N, 2048, N) == -6
    mu = lib.fp8_e4m3_gemv_multi
    mu.restype = I
    mu.argtypes = [P, L, I, I, I] + [P] * 7 + [P]
    PP = ctypes.c_void_p * 2
    ptrs = PP(None, None)
    Ns = (ctypes.c_int * 2)(1024, 512)
    strides = (ctypes.c_int64 * 2)(4096, 4096)
    assert mu(N, 4096, 4096, 1, 0, ptrs, ptrs, Ns, strides, strides, ptrs, strides, N) == -6   # n_mats < 1
    assert mu(N, 4096, 4096, 1, 9, ptrs, ptrs, Ns, strides, strides, ptrs, strides, N) == -6   # n_mats > 8
    assert mu(N, 4096, 4096, 1, 2, None, ptrs, Ns, strides, strides, ptrs, strides, N) == -6   # null table
    assert mu(N, 4096, 4000, 1, 2, ptrs, ptrs, Ns, strides, strides, ptrs, strides, N) == -1   # K % 128
    assert mu(N, 4096, 4096, 0, 2, ptrs, ptrs, Ns, strides, strides, ptrs, strides, N) == -5   # T < 1
    Ns[1] = 0
    assert mu(N, 4096, 4096, 1, 2, ptrs, ptrs, Ns, strides, strides, ptrs, strides, N) == -4   # N < 1
    fs = lib.fp8_e4m3_gemv_f32s
    fs.restype = I
    fs.argtypes = [P, L, P, P, I, I, I, L, L, P, L, P]
    assert fs(N, 4096, N, N, 4096, 1536, 0, 4096, 32, N, 1536, N) == -5          # T < 1
    assert fs(N, 4096, N, N, 4000, 1536, 1, 4096, 32, N, 1536, N) == -1          # K % 128
    assert fs(N, 4096, N, N, 16512, 1536, 1, 16512, 129, N, 1536, N) == -3       # K > 16384
    D4 = ctypes.c_void_p(1 << 20)
    assert fs(D4, 4096, D4, ctypes.c_void_p((1 << 20) + 2), 4096, 1536, 1, 4096, 32, D4, 1536, N) == -6  # misaligned
    assert fs(D4, 4096, D4, D4, 4096, 1536, 1, 4096, 31, D4, 1536, N) == -6      # scale row stride < K/128
    rn = lib.fp8_e4m3_rmsnorm_gemv
    rn.restype = I
    rn.argtypes = [P, P, P, ctypes.c_float, P, P, I, I, I, L, L, P, P, P, P]
    assert rn(N, N, N, 1e-6, N, N, 4096, 1536, 5, 4096, 32, N, N, N, N) == -5
    assert rn(N, N, N, 1e-6, N, N, 4000, 1536, 1, 4096, 32, N, N, N, N) == -1
    assert rn(N, N, N, 1e-6, N, N, 1024, 1536, 1, 1024, 8, N, N, N, N) == -6
    assert rn(N, N, N, 1e-6, N, N, 4096, 1536, 1, 4096, 32, N, None, N, N) == -6  # no x_norm


def test_fp8_and_dequant_extensions_reject_null_operands():
    """The FP8 extensions and the dense MXFP4 dequant return -10 when an
    operand pointer is null, after the shape checks and before any HIP call
    (one pointer null at a time; the others a 16-byte aligned address that is
    never dereferenced)."""
    fl = _lib("fp8-dense/libfp8_e4m3_gemv.so")
    P, I, L, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    D = ctypes.c_void_p(1 << 20)

    def each_null(fn, argtypes, build, n_ptr):
        fn.restype = I
        fn.argtypes = argtypes
        for i in range(n_ptr):
            ptrs = [D] * n_ptr
            ptrs[i] = N
            assert fn(*build(ptrs)) == -10, f"{fn.__name__}: pointer {i}"

    each_null(fl.fp8_e4m3_gemv, [P, L, P, P, I, I, I, L, L, P, L, P],
              lambda p: [p[0], 4096, p[1], p[2], 4096, 1536, 2, 4096, 32, p[3], 1536, N], 4)
    each_null(fl.fp8_e4m3_gemv_f32s, [P, L, P, P, I, I, I, L, L, P, L, P],
              lambda p: [p[0], 4096, p[1], p[2], 4096, 1536, 2, 4096, 32, p[3], 1536, N], 4)
    each_null(fl.fp8_e4m3_gemv_grouped, [P, L, L, P, P, I, I, I, I, L, L, P, L, L, P],
              lambda p: [p[0], 32768, 4096, p[1], p[2], 8, 4096, 1024, 1, 4096, 32, p[3], 8192, 1024, N], 4)
    each_null(fl.fp8_e4m3_swiglu_gemv, [P, L, P, P, P, P, I, I, I, L, L, F, I, P, L, P],
              lambda p: [p[0], 4096, p[1], p[2], p[3], p[4], 4096, 2048, 1, 4096, 32, 10.0, 1, p[5], 2048, N], 6)
    # x, W, S, y; norm_weight and x_norm set, no residual
    each_null(fl.fp8_e4m3_rmsnorm_gemv, [P, P, P, F, P, P, I, I, I, L, L, P, P, P, P],
              lambda p: [p[0], N, D, 1e-6, p[1], p[2], 4096, 1536, 1, 4096, 32, p[3], D, N, N], 4)
    each_null(fl.fp8_e4m3_dequant_bf16, [P, P, I, I, L, L, P, P],
              lambda p: [p[0], p[1], 4096, 1536, 4096, 32, p[2], N], 3)
    mu = fl.fp8_e4m3_gemv_multi
    mu.restype = I
    mu.argtypes = [P, L, I, I, I] + [P] * 7 + [P]
    Ns = (ctypes.c_int * 2)(1024, 512)
    strides = (ctypes.c_int64 * 2)(4096, 4096)
    full = (ctypes.c_void_p * 2)(1 << 20, 1 << 21)
    holed = (ctypes.c_void_p * 2)(1 << 20, None)
    assert mu(N, 4096, 4096, 1, 2, full, full, Ns, strides, strides, full, strides, N) == -10     # x
    assert mu(D, 4096, 4096, 1, 2, holed, full, Ns, strides, strides, full, strides, N) == -10    # W[1]
    assert mu(D, 4096, 4096, 1, 2, full, holed, Ns, strides, strides, full, strides, N) == -10    # S[1]
    assert mu(D, 4096, 4096, 1, 2, full, full, Ns, strides, strides, holed, strides, N) == -10    # y[1]
    ml = _lib("mxfp4-dense/libmxfp4_gemv.so")
    each_null(ml.mxfp4_dequant_bf16, [P, P, I, I, L, L, P, P],
              lambda p: [p[0], p[1], 4096, 2048, 2048, 128, p[2], N], 3)


def test_rmsnorm_validation_codes():
    lib = _lib("rmsnorm-fuse/librmsnorm_fuse.so")
    f = lib.rmsnorm_fuse_fwd
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 2 + [ctypes.c_float, ctypes.c_void_p]
    assert f(N, N, N, 0, 4096, 1e-6, N) == 0
    assert f(N, N, N, 4, 0, 1e-6, N) == 0
    assert f(N, N, N, 4, 8193, 1e-6, N) == 1
    g = lib.rmsnorm_fuse_residual_add
    g.restype = ctypes.c_int
    g.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 2 + [ctypes.c_float, ctypes.c_void_p]
    assert g(N, N, N, N, N, -1, 4096, 1e-6, N) == 0
    assert g(N, N, N, N, N, 4, 8193, 1e-6, N) == 1


def test_bindings_import_and_resolve_paths():
    from runtime import (fp8_e4m3_gemv_binding, mxfp4_gemv_binding, mxfp4_grouped_gemv_binding,
                         rmsnorm_fuse_binding)
    for mod, rel in ((mxfp4_grouped_gemv_binding, "mxfp4-routed/libmxfp4_grouped_gemv.so"),
                     (mxfp4_gemv_binding, "mxfp4-dense/libmxfp4_gemv.so"),
                     (fp8_e4m3_gemv_binding, "fp8-dense/libfp8_e4m3_gemv.so"),
                     (rmsnorm_fuse_binding, "rmsnorm-fuse/librmsnorm_fuse.so")):
        assert mod.lib_path() == os.path.join(PKG, "kernel", rel)
        mod._load_lib()  # sets argtypes for every exported entry point


def test_binding_env_override(monkeypatch, tmp_path):
    from runtime import mxfp4_gemv_binding

    monkeypatch.setenv("MXFP4_GEMV_LIB", str(tmp_path / "elsewhere.so"))
    assert mxfp4_gemv_binding.lib_path() == str(tmp_path / "elsewhere.so")


def test_bindings_reject_cpu_tensors():
    import torch

    from runtime import fp8_e4m3_gemv_binding, mxfp4_gemv_binding, mxfp4_grouped_gemv_binding
    from runtime import rmsnorm_fuse_binding

    x = torch.zeros(4096, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        mxfp4_gemv_binding.mxfp4_gemv(torch.zeros(8, 2048, dtype=torch.uint8),
                                      torch.zeros(8, 128, dtype=torch.uint8), x)
    with pytest.raises(RuntimeError):
        fp8_e4m3_gemv_binding.fp8_e4m3_gemv(torch.zeros(128, 4096, dtype=torch.uint8),
                                            torch.zeros(1, 32, dtype=torch.uint8), x)
    w = {"packed": torch.zeros(1, 32, 2048, dtype=torch.uint8),
         "scale": torch.zeros(1, 32, 128, dtype=torch.uint8)}
    with pytest.raises(ValueError):
        mxfp4_grouped_gemv_binding.mxfp4_grouped_gemv(w, w, w, None, x, torch.zeros(1))
    with pytest.raises(TypeError):
        rmsnorm_fuse_binding.rmsnorm_fuse_fwd(x.view(1, -1), x)
