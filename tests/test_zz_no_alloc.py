"""hkmoe_moe_forward_noalloc, the allocation-free layer, through the C ABI
(ctypes on libhkmoe.so) against hkmoe_moe_forward with a caller workspace.

Bar: bit-identical outputs (the same kernels; only the workspace differs), on
two calls in a row on the same device, the second with fewer tokens, in both
scale modes; with block scales these layers take the one-stream narrow
schedule, which must also match the layer with the narrow path switched off;
a layer whose workspace exceeds the library's scratch is refused on the host
with HKMOE_ERR_WORKSPACE.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "distributed-hipkittens_amd", "libhkmoe.so")
SCALE_TENSOR, SCALE_BLOCK = 0, 1
W_PACKED = 1
ERR_WORKSPACE = 4
H, I, E, K = 512, 256, 16, 4

i32, i64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p


@pytest.fixture(scope="module")
def lib(hk):
    lib = ctypes.CDLL(LIB)
    lib.hkmoe_last_error.restype = ctypes.c_char_p
    lib.hkmoe_moe_workspace_size.restype = ctypes.c_size_t
    return lib


def _p(t):
    return vp(t.data_ptr())


def _weights(hk, block, gen):
    if block:
        w13_q, w13_s = hk.quant_block(torch.randn((E, 2 * I, H), generator=gen, device="cuda"))
        w2_q, w2_s = hk.quant_block(torch.randn((E, H, I), generator=gen, device="cuda"))
    else:
        q13, s13, q2, s2 = [], [], [], []
        for _ in range(E):
            q, s = hk.quant_tensor(torch.randn((2 * I, H), generator=gen, device="cuda"))
            q13.append(q); s13.append(s)
            q, s = hk.quant_tensor(torch.randn((H, I), generator=gen, device="cuda"))
            q2.append(q); s2.append(s)
        w13_q, w13_s, w2_q, w2_s = torch.stack(q13), torch.cat(s13), torch.stack(q2), torch.cat(s2)
    return hk.pack_weights(w13_q, gate_up=True), w13_s, hk.pack_weights(w2_q), w2_s


def _tokens(hk, block, t, gen):
    x = torch.randn((t, H), generator=gen, device="cuda")
    x_q, x_s = hk.quant_group(x) if block else hk.quant_tensor(x)
    lg = torch.randn((t, E), generator=gen, device="cuda")
    rank = torch.randperm(E, generator=gen, device="cuda").float() + 1.0
    return x_q, x_s, (lg - 1.1 * torch.log(rank)[None, :]).contiguous()


def _forward(lib, w, tok, mode, t, out, ws=None):
    stream = vp(torch.cuda.current_stream().cuda_stream)
    args = [_p(tok[0]), _p(tok[1]), _p(tok[2]), _p(w[0]), _p(w[1]), _p(w[2]), _p(w[3]), i64(t), i32(E), i32(K),
            i32(H), i32(I), ctypes.c_int(mode), ctypes.c_int(W_PACKED), _p(out)]
    if ws is None:
        rc = lib.hkmoe_moe_forward_noalloc(*args, stream)
    else:
        rc = lib.hkmoe_moe_forward(*args, _p(ws), ctypes.c_size_t(ws.numel()), stream)
    assert rc == 0, lib.hkmoe_last_error().decode()


@pytest.mark.parametrize("block", [True, False])
def test_noalloc_matches_workspace_entry_point(hk, lib, block):
    gen = torch.Generator(device="cuda").manual_seed(900 + block)
    mode = SCALE_BLOCK if block else SCALE_TENSOR
    w = _weights(hk, block, gen)
    for t in (300, 70):  # the second call is smaller and reuses the scratch
        tok = _tokens(hk, block, t, gen)
        ws = torch.empty(lib.hkmoe_moe_workspace_size(i64(t), E, K, H, I, mode), dtype=torch.uint8, device="cuda")
        want = torch.empty((t, H), dtype=torch.bfloat16, device="cuda")
        got = torch.full((t, H), float("nan"), dtype=torch.bfloat16, device="cuda")
        _forward(lib, w, tok, mode, t, want, ws)
        _forward(lib, w, tok, mode, t, got)
        torch.cuda.synchronize()
        print(f"noalloc block={block} T={t}: max|out|={want.float().abs().max().item():.3f}", flush=True)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        # the same layer without the narrow kernels (256x256 tiles only)
        saved = hk.tk_kernel.get_narrow()
        wide = torch.full((t, H), float("nan"), dtype=torch.bfloat16, device="cuda")
        try:
            hk.tk_kernel.set_narrow(0, saved[1], saved[2])
            _forward(lib, w, tok, mode, t, wide)
            torch.cuda.synchronize()
        finally:
            hk.tk_kernel.set_narrow(*saved)
        assert torch.equal(got.view(torch.int16), wide.view(torch.int16))


def test_noalloc_rejects_layers_beyond_the_scratch(hk, lib):
    fake = vp(0x1000)  # never dereferenced: the size check comes first
    t = 4096
    need = lib.hkmoe_moe_workspace_size(i64(t), 256, 8, 7168, 2048, SCALE_BLOCK)
    assert need > (64 << 20)
    rc = lib.hkmoe_moe_forward_noalloc(fake, fake, fake, fake, fake, fake, fake, i64(t), i32(256), i32(8),
                                       i32(7168), i32(2048), ctypes.c_int(SCALE_BLOCK), ctypes.c_int(W_PACKED),
                                       fake, vp(0))
    assert rc == ERR_WORKSPACE
    assert "scratch" in lib.hkmoe_last_error().decode()
