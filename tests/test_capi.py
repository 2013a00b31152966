"""C ABI and binding checks that need no GPU: the library loads, exports every
entry point include/hkmoe.h declares, rejects bad arguments on the host
before touching the device, and sizes the layer workspace as documented."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hkmoe.h")
# HKMOE_LIB: another build of the same library (the host-sanitizer run loads one)
LIB = os.environ.get("HKMOE_LIB") or os.path.join(ROOT, "distributed-hipkittens_amd", "libhkmoe.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hkmoe_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libhkmoe.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB)
    lib.hkmoe_last_error.restype = ctypes.c_char_p
    lib.hkmoe_moe_workspace_size.restype = ctypes.c_size_t
    return lib


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 14, names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_version(lib):
    assert lib.hkmoe_version() >= 100


def _err(lib):
    return lib.hkmoe_last_error().decode()


def test_gemm_argument_errors_are_host_side(lib):
    i64 = ctypes.c_int64
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    assert lib.hkmoe_gemm_fp8(None, fake, fake, i64(64), i64(256), i64(128), None, None, 0, None) == 1
    assert "null" in _err(lib)
    assert lib.hkmoe_gemm_fp8(fake, fake, fake, i64(64), i64(256), i64(100), None, None, 0, None) == 1
    assert "multiple of 128" in _err(lib)
    assert lib.hkmoe_gemm_fp8(fake, fake, fake, i64(64), i64(200), i64(128), None, None, 0, None) == 1
    assert "multiple of 256" in _err(lib)
    assert lib.hkmoe_gemm_fp8(fake, fake, fake, i64(64), i64(256), i64(128), None, None, 7, None) == 1
    assert "out_dtype" in _err(lib)
    # A of 4 GiB or more cannot be addressed by 32-bit buffer offsets: refused
    # (M = 8192, N = 256, K = 2^20 would take the 128x128 path with M*K = 2^33)
    assert lib.hkmoe_gemm_fp8(fake, fake, fake, i64(8192), i64(256), i64(1 << 20), None, None, 0, None) == 1
    assert "M*K" in _err(lib)
    assert lib.hkmoe_gemm_fp8(fake, fake, fake, i64(1 << 22), i64(256), i64(1024), None, None, 0, None) == 1
    assert "M*K" in _err(lib)


def test_dense_mfma_setting(lib):
    saved = lib.hkmoe_get_dense_mfma()
    assert saved in (16, 32)
    assert lib.hkmoe_set_dense_mfma(ctypes.c_int32(8)) == 1
    assert "16 or 32" in _err(lib)
    assert lib.hkmoe_set_dense_mfma(ctypes.c_int32(32)) == 0 and lib.hkmoe_get_dense_mfma() == 32
    assert lib.hkmoe_set_dense_mfma(ctypes.c_int32(saved)) == 0


def test_kernel_timing_argument_errors(lib):
    f = (ctypes.c_float * 16)()
    assert lib.hkmoe_kernel_timing(ctypes.c_int32(-1)) == 1
    assert lib.hkmoe_kernel_timing(ctypes.c_int32(0)) == 0  # off: no device work
    assert lib.hkmoe_kernel_timing_read(ctypes.c_int32(0), f, f, ctypes.c_int32(16)) == 1
    assert "outside" in _err(lib)
    assert lib.hkmoe_kernel_timing_read(ctypes.c_int32(0), f, f, ctypes.c_int32(3)) == 1


def test_routing_argument_errors(lib):
    fake = ctypes.c_void_p(0x1000)
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    assert lib.hkmoe_route_topk(fake, i64(16), i32(2000), i32(2), fake, fake, fake, None) == 1
    assert "E=2000" in _err(lib)
    assert lib.hkmoe_route_topk(fake, i64(16), i32(8), i32(9), fake, fake, fake, None) == 1
    assert "top_k=9" in _err(lib)
    assert lib.hkmoe_route_topk(fake, i64(16), i32(64), i32(33), fake, fake, fake, None) == 1
    assert lib.hkmoe_combine(fake, fake, fake, i64(4), i32(2), i32(100), fake, None) == 1
    assert "multiple of 8" in _err(lib)


def test_moe_forward_argument_errors(lib):
    fake = ctypes.c_void_p(0x1000)
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    args = [fake] * 7 + [i64(64), i32(8), i32(2), i32(4096), i32(1024), 0, 0, fake, None, ctypes.c_size_t(0),
                         None]
    assert lib.hkmoe_moe_forward(*args) == 4  # HKMOE_ERR_WORKSPACE
    assert "workspace" in _err(lib)
    args[12] = 2  # bad scale mode
    assert lib.hkmoe_moe_forward(*args) == 1
    assert "scale_mode" in _err(lib)
    args[12] = 0
    args[13] = 3  # bad weight layout
    assert lib.hkmoe_moe_forward(*args) == 1
    assert "w_layout" in _err(lib)
    args[13] = 0
    args[10] = i32(4000)  # hidden not a multiple of 256
    assert lib.hkmoe_moe_forward(*args) == 1
    assert "hidden=4000" in _err(lib)
    args[10] = i32(4096)
    args[11] = i32(16512)  # I beyond GEMM 2's 128 K steps: refused before any launch
    assert lib.hkmoe_moe_forward(*args) == 1
    assert "inter=16512" in _err(lib)
    # hq = T*k rows of I bytes past 4 GiB cannot be addressed by 32-bit buffer
    # offsets: refused before any launch (T*k*I = 2^19 * 8 * 1024 = 2^32)
    args[7], args[8], args[9], args[11] = i64(1 << 19), i32(64), i32(8), i32(1024)
    assert lib.hkmoe_moe_forward(*args) == 1
    assert "T*k*I" in _err(lib)
    mx = args[:12] + [0, fake, fake, ctypes.c_size_t(1 << 40), None]
    assert lib.hkmoe_moe_forward_mx(*mx) == 1
    assert "T*k*I" in _err(lib)
    # the same bound on the stepwise GEMM 2 (rows*I = 2^22 * 1024)
    rc = lib.hkmoe_grouped_gemm2(fake, fake, fake, fake, fake, fake, None, i64(1 << 22), i32(8), i32(256),
                                 i32(1024), 1, 0, fake, None, None)
    assert rc == 1 and "rows*inter" in _err(lib)


def test_moe_forward_empty_batch(lib):
    """T = 0: nothing is launched (no GPU needed); activations, output and
    workspace may be null, the weights and shapes are still checked."""
    fake = ctypes.c_void_p(0x1000)
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    shape = [i64(0), i32(8), i32(2), i32(4096), i32(1024)]
    args = [None, None, None, fake, fake, fake, fake] + shape + [1, 0, None, None, ctypes.c_size_t(0), None]
    assert lib.hkmoe_moe_forward(*args) == 0
    noalloc = [None, None, None, fake, fake, fake, fake] + shape + [1, 0, None, None]
    assert lib.hkmoe_moe_forward_noalloc(*noalloc) == 0
    mx = [None, None, None, fake, fake, fake, fake] + shape + [1, None, None, ctypes.c_size_t(0), None]
    assert lib.hkmoe_moe_forward_mx(*mx) == 0
    args[3] = None  # the weights are still required
    assert lib.hkmoe_moe_forward(*args) == 1
    assert "null pointer" in _err(lib)
    args[3] = fake
    args[10] = i32(4000)  # and the shapes checked
    assert lib.hkmoe_moe_forward(*args) == 1
    assert "hidden=4000" in _err(lib)
    args[10] = i32(4096)
    args[7] = i64(64)  # with tokens, null activations are an error
    assert lib.hkmoe_moe_forward(*args) == 1
    assert "null pointer" in _err(lib)


def test_grouped_gemm_format_errors(lib):
    fake = ctypes.c_void_p(0x1000)
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    # e4m3 intermediate output is only defined for block scales
    rc = lib.hkmoe_grouped_gemm1(fake, fake, fake, i32(2), i64(64), fake, fake, fake, fake, None, i64(128),
                                 i32(8), i32(256), i32(128), 0, 0, 2, fake, fake, None, None)
    assert rc == 1 and "out_format" in _err(lib)
    rc = lib.hkmoe_grouped_gemm1(fake, fake, fake, i32(2), i64(64), fake, fake, fake, fake, None, i64(128),
                                 i32(8), i32(256), i32(96), 1, 0, 0, fake, fake, None, None)
    assert rc == 1 and "inter=96" in _err(lib)
    rc = lib.hkmoe_grouped_gemm1(fake, fake, fake, i32(2), i64(64), fake, fake, fake, fake, None, i64(128),
                                 i32(8), i32(256), i32(128), 1, 5, 0, fake, fake, None, None)
    assert rc == 1 and "w_layout" in _err(lib)
    rc = lib.hkmoe_grouped_gemm2(fake, fake, fake, fake, fake, fake, None, i64(128), i32(8), i32(256), i32(128),
                                 1, 2, fake, None, None)
    assert rc == 1 and "w_layout" in _err(lib)


def test_narrow_split_argument_errors(lib):
    """The narrow split entry points reject bad arguments on the host (before
    any launch): no narrow_info or M-tile list, a bad part, odd K-step counts,
    a row threshold above 64 and out-of-range settings."""
    fake = ctypes.c_void_p(0x1000)
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    g1 = lambda ni, ml, part, hidden: lib.hkmoe_grouped_gemm1_part(
        fake, fake, fake, i32(2), i64(64), fake, fake, fake, fake, ml, i64(128), i32(8), i32(hidden), i32(128),
        1, fake, fake, None, ni, i32(part), i32(0), None)
    assert g1(None, fake, 1, 256) == 1 and "narrow_info" in _err(lib)
    assert g1(fake, None, 1, 256) == 1 and "mtile_list" in _err(lib)
    assert g1(fake, fake, 2, 256) == 1 and "part=2" in _err(lib)
    assert g1(fake, fake, 1, 384) == 1 and "H=384" in _err(lib)
    rc = lib.hkmoe_grouped_gemm2_part(fake, fake, fake, fake, fake, fake, fake, i64(128), i32(8), i32(256),
                                      i32(384), 1, fake, None, fake, i32(1), i32(0), None)
    assert rc == 1 and "I=384" in _err(lib)
    rc = lib.hkmoe_expert_offsets_narrow(fake, i64(64), i32(8), fake, fake, fake, fake, fake, None, None,
                                         i32(65), fake, None)
    assert rc == 1 and "narrow_max=65" in _err(lib)
    assert lib.hkmoe_set_narrow(i32(-1), i32(64), i32(0)) == 1
    assert lib.hkmoe_set_narrow(i32(8), i32(65), i32(0)) == 1
    assert lib.hkmoe_set_narrow(i32(8), i32(64), i32(3)) == 1 and "wide_share=3" in _err(lib)
    c, r, w = i32(), i32(), i32()
    assert lib.hkmoe_get_narrow(ctypes.byref(c), ctypes.byref(r), ctypes.byref(w)) == 0
    assert 0 <= c.value and 0 <= r.value <= 64


def test_pack_weights_argument_errors(lib):
    fake, other = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000)
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    assert lib.hkmoe_pack_weights(fake, i64(4), i64(384), i64(256), i32(0), other, None) == 1
    assert "N=384" in _err(lib)
    assert lib.hkmoe_pack_weights(fake, i64(4), i64(512), i64(192), i32(0), other, None) == 1
    assert lib.hkmoe_pack_weights(fake, i64(4), i64(512), i64(256), i32(128), other, None) == 1
    assert "gate_up=128" in _err(lib)
    assert lib.hkmoe_pack_weights(fake, i64(4), i64(512), i64(256), i32(0), fake, None) == 1
    assert "in-place" in _err(lib)
    # nothing to do for zero experts: succeeds without touching the GPU
    assert lib.hkmoe_pack_weights(fake, i64(0), i64(512), i64(256), i32(256), other, None) == 0


def test_mx_argument_errors(lib):
    fake = ctypes.c_void_p(0x1000)
    i64 = ctypes.c_int64
    assert lib.hkmoe_quant_mx(fake, i64(4), i64(48), fake, fake, None) == 1
    assert "multiple of 32" in _err(lib)
    assert lib.hkmoe_quant_mx(None, i64(4), i64(64), fake, fake, None) == 1
    assert lib.hkmoe_quant_mx(fake, i64(0), i64(64), fake, fake, None) == 0  # empty: no launch
    assert lib.hkmoe_mx_pack_scales(fake, i64(4), i64(96), fake, None) == 1
    assert "multiple of 128" in _err(lib)
    assert lib.hkmoe_gemm_mx(fake, fake, fake, fake, fake, i64(64), i64(256), i64(96), 1, None) == 1
    assert "multiple of 128" in _err(lib)
    assert lib.hkmoe_gemm_mx(fake, fake, fake, fake, fake, i64(64), i64(320), i64(128), 1, None) == 1
    assert "multiple of 256" in _err(lib)
    assert lib.hkmoe_gemm_mx(fake, None, fake, fake, fake, i64(64), i64(256), i64(128), 1, None) == 1
    assert "null" in _err(lib)
    assert lib.hkmoe_gemm_mx(fake, fake, fake, fake, fake, i64(64), i64(256), i64(128), 5, None) == 1
    assert "out_dtype" in _err(lib)
    assert lib.hkmoe_gemm_mx(fake, fake, fake, fake, fake, i64(1 << 22), i64(256), i64(1024), 1, None) == 1
    assert "M*K" in _err(lib)
    assert lib.hkmoe_gemm_mx(fake, fake, fake, fake, fake, i64(0), i64(256), i64(128), 1, None) == 0


def test_mx_moe_argument_errors(lib):
    fake, other = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000)
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    lib.hkmoe_mx_words_per_step.restype = ctypes.c_int64
    assert lib.hkmoe_mx_words_per_step(i64(65536), i32(256)) == (256 + 256) * 256
    assert lib.hkmoe_mx_words_per_step(i64(1), i32(4)) == (1 + 4) * 256
    assert lib.hkmoe_moe_workspace_size(i64(64), 8, 2, 256, 128, 7) == 0  # unknown scale mode
    assert lib.hkmoe_moe_workspace_size(i64(64), 8, 2, 256, 128, 2) > 0   # HKMOE_SCALE_MX
    assert lib.hkmoe_mx_pack_weight_scales(fake, i64(2), i64(384), i64(256), i32(0), other, None) == 1
    assert "multiple of 256" in _err(lib)
    assert lib.hkmoe_mx_pack_weight_scales(fake, i64(2), i64(512), i64(256), i32(128), other, None) == 1
    assert "gate_up" in _err(lib)
    rc = lib.hkmoe_grouped_gemm1_mx(fake, fake, fake, i32(2), i64(64), fake, fake, fake, fake, None, i64(128),
                                    i32(8), i32(256), i32(128), 1, 9, fake, fake, None, None)
    assert rc == 1 and "out_format" in _err(lib)
    rc = lib.hkmoe_grouped_gemm2_mx(fake, fake, fake, fake, fake, fake, None, i64(128), i32(8), i32(200),
                                    i32(128), 1, fake, None, None)
    assert rc == 1 and "multiple of 256" in _err(lib)
    ws = lib.hkmoe_moe_workspace_size(i64(64), 8, 2, 256, 128, 2)
    args = [fake, fake, fake, fake, fake, fake, fake, i64(64), i32(8), i32(2), i32(256), i32(128), 1, fake,
            fake, ctypes.c_size_t(ws - 1), None]
    assert lib.hkmoe_moe_forward_mx(*args) == 4  # HKMOE_ERR_WORKSPACE


def _align(x):
    return (x + 255) // 256 * 256


@pytest.mark.parametrize("t,e,k,h,i,block", [(8192, 256, 8, 7168, 2048, True), (4096, 8, 2, 4096, 14336, False),
                                             (64, 128, 8, 4096, 1536, True), (0, 4, 1, 256, 128, True)])
def test_workspace_size_formula(lib, t, e, k, h, i, block):
    r = t * k
    nblk = (t + 31) // 32
    parts = [r * 4, r * 4, nblk * e * 4, nblk * e * 4, e * 4, (e + 1) * 4, (e + 1) * 4,
             ((r + 255) // 256 + e) * 8, 4, 16 * 4, 5 * 4, r * 4, r * 4]
    if not block:
        parts.append(r * i * 2)
    parts += [r * i, r * (i // 128) * 4 if block else 4, r * h * 2]
    want = sum(_align(p) for p in parts)
    got = lib.hkmoe_moe_workspace_size(ctypes.c_int64(t), ctypes.c_int32(e), ctypes.c_int32(k),
                                       ctypes.c_int32(h), ctypes.c_int32(i), 1 if block else 0)
    assert got == want


def test_pybind_module_rejects_host_tensors():
    import sys
    import torch
    sys.path.insert(0, os.path.join(ROOT, "distributed-hipkittens_amd"))
    import tk_kernel
    a = torch.zeros((256, 128), dtype=torch.float8_e4m3fn)
    c = torch.zeros((256, 256), dtype=torch.float32)
    with pytest.raises(RuntimeError, match="GPU device"):
        tk_kernel.dispatch_micro(a, a, c)
    with pytest.raises(RuntimeError, match="torch.Tensor"):
        tk_kernel.dispatch_micro(c.numpy(), a, c)
    assert tk_kernel.route_blocks(8192) == 256
