"""MoE layer orchestration over the tk_kernel dispatch entry points.

Torch is used only for device memory (allocation of outputs and the
workspace) and for the current stream; every operation is one of the HIP
kernels behind ``tk_kernel``.
"""
import torch

import tk_kernel

F8 = torch.float8_e4m3fn
GROUP = 128


def _check_dev(*ts):
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("hkmoe: tensors must live on a GPU device")


# ----------------------------------------------------------------------------
# quantisers (device)
# ----------------------------------------------------------------------------
def quant_group(x):
    """fp32 [R, C] -> (e4m3 [R, C], fp32 scales [R, C/128]), 1x128 groups."""
    _check_dev(x)
    x = x.float().contiguous()
    q = torch.empty(x.shape, dtype=F8, device=x.device)
    s = torch.empty((x.shape[0], x.shape[1] // GROUP), dtype=torch.float32, device=x.device)
    tk_kernel.dispatch_quant_group(x, q, s)
    return q, s


def quant_block(w):
    """fp32 [..., R, C] -> (e4m3, fp32 scales [..., R/128, C/128]), 128x128 blocks."""
    _check_dev(w)
    w = w.float().contiguous()
    q = torch.empty(w.shape, dtype=F8, device=w.device)
    s = torch.empty((*w.shape[:-2], w.shape[-2] // GROUP, w.shape[-1] // GROUP),
                    dtype=torch.float32, device=w.device)
    tk_kernel.dispatch_quant_block(w.reshape(-1, w.shape[-2], w.shape[-1]), q, s)
    return q, s


def quant_tensor(x):
    """fp32 tensor -> (e4m3, fp32 scale [1]), s = amax/448."""
    _check_dev(x)
    x = x.float().contiguous()
    q = torch.empty(x.shape, dtype=F8, device=x.device)
    s = torch.empty(1, dtype=torch.float32, device=x.device)
    ws = torch.empty(1, dtype=torch.float32, device=x.device)
    tk_kernel.dispatch_quant_tensor(x, q, s, ws)
    return q, s


def gemm_fp8(a_q, b_q, scale_a=None, scale_b=None, out_dtype=torch.bfloat16):
    """C = (sa*sb) A . B^T for e4m3 A [M,K], B [N,K]."""
    _check_dev(a_q, b_q)
    c = torch.empty((a_q.shape[0], b_q.shape[0]), dtype=out_dtype, device=a_q.device)
    tk_kernel.dispatch_gemm_fp8(a_q, b_q, c, scale_a, scale_b)
    return c


# ----------------------------------------------------------------------------
# MX (1x32 e8m0) operands and GEMM
# ----------------------------------------------------------------------------
def quant_mx(x):
    """fp32 [R, C] -> (e4m3 [R, C], e8m0 exponents uint8 [R, C/32])."""
    _check_dev(x)
    x = x.float().contiguous()
    q = torch.empty(x.shape, dtype=F8, device=x.device)
    s = torch.empty((x.shape[0], x.shape[1] // 32), dtype=torch.uint8, device=x.device)
    tk_kernel.dispatch_quant_mx(x, q, s)
    return q, s


def mx_pack_scales(s):
    """e8m0 exponents uint8 [R, C/32] -> packed MFMA words int32 [C/128, R64]."""
    _check_dev(s)
    s = s.contiguous()
    rows, cols = s.shape[0], s.shape[1] * 32
    packed = torch.empty((cols // 128, (rows + 63) // 64 * 64), dtype=torch.int32, device=s.device)
    tk_kernel.dispatch_mx_pack_scales(s, cols, packed)
    return packed


def gemm_mx(a_q, a_packed, b_q, b_packed, out_dtype=torch.float32):
    """C = A . B^T with 1x32 e8m0 block scales (packed by mx_pack_scales)."""
    _check_dev(a_q, b_q)
    c = torch.empty((a_q.shape[0], b_q.shape[0]), dtype=out_dtype, device=a_q.device)
    tk_kernel.dispatch_gemm_mx(a_q, a_packed, b_q, b_packed, c)
    return c


# ----------------------------------------------------------------------------
# the layer
# ----------------------------------------------------------------------------
def pack_weights(w_q, gate_up=False):
    """Load-time repack of e4m3 expert weights [E, N, K] into the grouped
    GEMMs' tile layout (hkmoe_pack_weights); same shape, new tensor.  Pass
    ``gate_up=True`` for the fused gate/up weights [E, 2I, H] of GEMM 1."""
    _check_dev(w_q)
    if w_q.dtype != F8 or w_q.dim() != 3:
        raise RuntimeError("pack_weights: expected float8_e4m3fn [E, N, K]")
    w_q = w_q.contiguous()
    packed = torch.empty_like(w_q)
    tk_kernel.dispatch_pack_weights(w_q, packed, w_q.shape[1] // 2 if gate_up else 0)
    return packed


def moe_forward(x_q, x_scale, logits, w13_q, w13_scale, w2_q, w2_scale, top_k,
                out=None, workspace=None, packed=False):
    """Single-call layer (hkmoe_moe_forward).  Returns the bf16 [T, H] output.
    ``packed``: w13_q / w2_q come from :func:`pack_weights`."""
    _check_dev(x_q, logits, w13_q, w2_q)
    t, hidden = x_q.shape
    e, two_i, _ = w13_q.shape
    mode = tk_kernel.SCALE_TENSOR if x_scale.numel() == 1 and x_scale.dim() <= 1 else tk_kernel.SCALE_BLOCK
    if out is None:
        out = torch.empty((t, hidden), dtype=torch.bfloat16, device=x_q.device)
    need = tk_kernel.moe_workspace_size(t, e, top_k, hidden, two_i // 2, mode)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x_q.device)
    tk_kernel.dispatch_moe(x_q, x_scale, logits, w13_q, w13_scale, w2_q, w2_scale, top_k, out,
                           workspace, packed=packed)
    return out


def moe_forward_steps(x_q, x_scale, logits, w13_q, w13_scale, w2_q, w2_scale, top_k,
                      keep_h=False, packed=False, narrow=None):
    """The layer one kernel at a time (the same kernels hkmoe_moe_forward
    enqueues); returns a dict of every intermediate.  With ``keep_h`` the block
    path also runs GEMM 1 once more with a bf16 output (``h``) for inspection.
    ``narrow = (cus, max_rows, share)`` (block scales) splits both GEMMs like
    hkmoe_moe_forward's narrow path: the experts of <= max_rows rows run in the
    narrow kernel on ``cus`` workgroups on a side stream (``r["side"]``), the
    others in the 256x256 kernel on the current stream (on CUs - cus
    workgroups for GEMM 1 with ``share``)."""
    _check_dev(x_q, logits, w13_q, w2_q)
    dev = x_q.device
    t, hidden = x_q.shape
    e, two_i, _ = w13_q.shape
    inter = two_i // 2
    rows = t * top_k
    block = not (x_scale.numel() == 1 and x_scale.dim() <= 1)
    i32 = dict(dtype=torch.int32, device=dev)
    f32 = dict(dtype=torch.float32, device=dev)
    nblk = tk_kernel.route_blocks(t)
    r = dict(
        topk_idx=torch.empty((t, top_k), **i32), topk_w=torch.empty((t, top_k), **f32),
        block_counts=torch.empty((nblk, e), **i32), block_base=torch.empty((nblk, e), **i32),
        counts=torch.empty(e, **i32), offsets=torch.empty(e + 1, **i32),
        mtile_offsets=torch.empty(e + 1, **i32), amax=torch.empty(1, **f32),
        mtile_list=torch.empty(tk_kernel.mtile_list_ints(t * min(e, 32), e), **i32),
        tile_ctr=torch.empty(16, **i32),
        perm=torch.empty(rows, **i32), inv_perm=torch.empty(rows, **i32),
        hq=torch.empty((rows, inter), dtype=F8, device=dev),
        hs=(torch.empty((inter // GROUP, rows), **f32) if block else torch.empty(1, **f32)),
        y=torch.empty((rows, hidden), dtype=torch.bfloat16, device=dev),
        out=torch.empty((t, hidden), dtype=torch.bfloat16, device=dev),
    )
    if not block or keep_h:
        r["h"] = torch.empty((rows, inter), dtype=torch.bfloat16, device=dev)
    if narrow is not None:
        if not block:
            raise RuntimeError("moe_forward_steps: the narrow split needs block scales")
        return _steps_narrow(r, x_q, x_scale, logits, w13_q, w13_scale, w2_q, w2_scale, top_k, packed,
                             narrow)
    tk_kernel.dispatch_route_topk(logits, r["topk_idx"], r["topk_w"], r["block_counts"])
    tk_kernel.dispatch_expert_offsets(r["block_counts"], t, r["counts"], r["offsets"],
                                      r["block_base"], r["mtile_offsets"], r["amax"], r["tile_ctr"],
                                      r["mtile_list"])
    tk_kernel.dispatch_scatter(r["topk_idx"], r["offsets"], r["block_base"], r["perm"],
                               r["inv_perm"], None, None, None, None)
    if block:
        tk_kernel.dispatch_grouped_gemm1(x_q, x_scale, r["perm"], top_k, w13_q, w13_scale,
                                         r["offsets"], r["mtile_offsets"], r["hq"], r["hs"],
                                         r["tile_ctr"][:8], packed=packed, mtile_list=r["mtile_list"])
        if keep_h:  # static tile order for the inspection pass
            tk_kernel.dispatch_grouped_gemm1(x_q, x_scale, r["perm"], top_k, w13_q, w13_scale,
                                             r["offsets"], r["mtile_offsets"], r["h"], None,
                                             packed=packed)
    else:
        tk_kernel.dispatch_grouped_gemm1(x_q, x_scale, r["perm"], top_k, w13_q, w13_scale,
                                         r["offsets"], r["mtile_offsets"], r["h"], r["amax"],
                                         r["tile_ctr"][:8], packed=packed, mtile_list=r["mtile_list"])
        tk_kernel.dispatch_requant(r["h"], r["amax"], r["hq"], r["hs"])
    tk_kernel.dispatch_grouped_gemm2(r["hq"], r["hs"], w2_q, w2_scale, r["offsets"],
                                     r["mtile_offsets"], r["y"], r["tile_ctr"][8:],
                                     packed=packed, mtile_list=r["mtile_list"])
    tk_kernel.dispatch_combine(r["y"], r["topk_w"], r["inv_perm"], r["out"])
    return r


def narrow_cus(cus, n_cu):
    """Workgroups the narrow kernels take while 256x256 tiles exist, as
    hkmoe_moe_forward limits them: at most three quarters of the CUs.  Both
    narrow kernels launch one workgroup per CU and the device lifts the limit
    when every expert is narrow, so passing this as ``grid`` of the part-1
    dispatches gives hkmoe_moe_forward's schedule; the first 256x256 GEMM then
    runs on ``n_cu - cus`` workgroups (wide_share >= 1)."""
    return min(cus, n_cu - n_cu // 4)


def _steps_narrow(r, x_q, x_scale, logits, w13_q, w13_scale, w2_q, w2_scale, top_k, packed, narrow):
    cus, max_rows, share = narrow
    t = x_q.shape[0]
    dev = x_q.device
    r["narrow_info"] = torch.zeros(5, dtype=torch.int32, device=dev)
    tk_kernel.dispatch_route_topk(logits, r["topk_idx"], r["topk_w"], r["block_counts"])
    tk_kernel.dispatch_expert_offsets(r["block_counts"], t, r["counts"], r["offsets"],
                                      r["block_base"], r["mtile_offsets"], r["amax"], r["tile_ctr"],
                                      r["mtile_list"], narrow_max=max_rows, narrow_info=r["narrow_info"])
    tk_kernel.dispatch_scatter(r["topk_idx"], r["offsets"], r["block_base"], r["perm"],
                               r["inv_perm"], None, None, None, None)
    main = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(main)
    split = dict(packed=packed, mtile_list=r["mtile_list"], narrow_info=r["narrow_info"])
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    cus = narrow_cus(cus, n_cu)
    with torch.cuda.stream(side):
        tk_kernel.dispatch_grouped_gemm1(x_q, x_scale, r["perm"], top_k, w13_q, w13_scale, r["offsets"],
                                         r["mtile_offsets"], r["hq"], r["hs"], None, part=1, grid=cus, **split)
        tk_kernel.dispatch_grouped_gemm2(r["hq"], r["hs"], w2_q, w2_scale, r["offsets"], r["mtile_offsets"],
                                         r["y"], None, part=1, grid=cus, **split)
    tk_kernel.dispatch_grouped_gemm1(x_q, x_scale, r["perm"], top_k, w13_q, w13_scale, r["offsets"],
                                     r["mtile_offsets"], r["hq"], r["hs"], r["tile_ctr"][:8], part=0,
                                     grid=n_cu - cus if share else 0, **split)
    tk_kernel.dispatch_grouped_gemm2(r["hq"], r["hs"], w2_q, w2_scale, r["offsets"], r["mtile_offsets"],
                                     r["y"], r["tile_ctr"][8:], part=0, grid=0, **split)
    main.wait_stream(side)
    tk_kernel.dispatch_combine(r["y"], r["topk_w"], r["inv_perm"], r["out"])
    r["side"] = side
    return r


class MoELayer:
    """FP8 MoE FFN layer: e4m3 expert weights with per-tensor ([E]) or
    128x128 block scales; runs hkmoe_moe_forward with a cached workspace.
    With ``pack`` (default) the weights are repacked once, here, into the
    grouped GEMMs' tile layout; the layer then holds only the packed copies."""

    def __init__(self, w13_q, w13_scale, w2_q, w2_scale, top_k, pack=True):
        _check_dev(w13_q, w2_q)
        if w13_q.dtype != F8 or w2_q.dtype != F8:
            raise RuntimeError("MoELayer: weights must be float8_e4m3fn")
        self.packed = bool(pack)
        if self.packed:
            self.w13_q, self.w2_q = pack_weights(w13_q, gate_up=True), pack_weights(w2_q)
        else:
            self.w13_q, self.w2_q = w13_q.contiguous(), w2_q.contiguous()
        self.w13_scale, self.w2_scale = w13_scale.contiguous(), w2_scale.contiguous()
        self.top_k = int(top_k)
        self.num_experts, two_i, self.hidden = w13_q.shape
        self.inter = two_i // 2
        self.block = w13_scale.dim() == 3
        self._ws = None

    def workspace(self, num_tokens, device):
        mode = tk_kernel.SCALE_BLOCK if self.block else tk_kernel.SCALE_TENSOR
        need = tk_kernel.moe_workspace_size(num_tokens, self.num_experts, self.top_k, self.hidden,
                                            self.inter, mode)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=device)
        return self._ws

    def __call__(self, x_q, x_scale, logits, out=None):
        ws = self.workspace(x_q.shape[0], x_q.device)
        return moe_forward(x_q, x_scale, logits, self.w13_q, self.w13_scale, self.w2_q,
                           self.w2_scale, self.top_k, out=out, workspace=ws, packed=self.packed)


# ----------------------------------------------------------------------------
# MX (1x32 e8m0) MoE layer
# ----------------------------------------------------------------------------
def mx_pack_weight_scales(s, gate_up=False):
    """e8m0 weight exponents uint8 [E, N, K/32] -> the grouped MX GEMMs' words
    (int32, [E, N/256, K/128, 256]); ``gate_up`` for the fused w13 [E, 2I, H/32]."""
    _check_dev(s)
    s = s.contiguous()
    e, n, kb = s.shape
    words = torch.empty((e, n // 256, kb // 4, 256), dtype=torch.int32, device=s.device)
    tk_kernel.dispatch_mx_pack_weight_scales(s, words, n // 2 if gate_up else 0)
    return words


def moe_forward_mx_steps(x_q, x_e8m0, logits, w13_q, w13_words, w2_q, w2_words, top_k,
                         keep_h=False, packed=False):
    """The MX layer one kernel at a time; returns every intermediate (``xw``:
    gathered activation words, ``hq``/``hw``: GEMM 1's e4m3 output and its
    words; with ``keep_h`` also GEMM 1's bf16 h)."""
    _check_dev(x_q, x_e8m0, logits, w13_q, w2_q)
    dev = x_q.device
    t, hidden = x_q.shape
    e, two_i, _ = w13_q.shape
    inter = two_i // 2
    rows = t * top_k
    ws = tk_kernel.mx_words_per_step(rows, e)
    i32 = dict(dtype=torch.int32, device=dev)
    f32 = dict(dtype=torch.float32, device=dev)
    nblk = tk_kernel.route_blocks(t)
    r = dict(
        topk_idx=torch.empty((t, top_k), **i32), topk_w=torch.empty((t, top_k), **f32),
        block_counts=torch.empty((nblk, e), **i32), block_base=torch.empty((nblk, e), **i32),
        counts=torch.empty(e, **i32), offsets=torch.empty(e + 1, **i32),
        mtile_offsets=torch.empty(e + 1, **i32), amax=torch.empty(1, **f32),
        mtile_list=torch.empty(tk_kernel.mtile_list_ints(t * min(e, 32), e), **i32),
        tile_ctr=torch.empty(16, **i32),
        perm=torch.empty(rows, **i32), inv_perm=torch.empty(rows, **i32),
        xw=torch.empty((hidden // GROUP, ws), **i32),
        hq=torch.empty((rows, inter), dtype=F8, device=dev),
        hw=torch.empty((inter // GROUP, ws), **i32),
        y=torch.empty((rows, hidden), dtype=torch.bfloat16, device=dev),
        out=torch.empty((t, hidden), dtype=torch.bfloat16, device=dev),
    )
    tk_kernel.dispatch_route_topk(logits, r["topk_idx"], r["topk_w"], r["block_counts"])
    tk_kernel.dispatch_expert_offsets(r["block_counts"], t, r["counts"], r["offsets"],
                                      r["block_base"], r["mtile_offsets"], r["amax"], r["tile_ctr"],
                                      r["mtile_list"])
    tk_kernel.dispatch_scatter(r["topk_idx"], r["offsets"], r["block_base"], r["perm"],
                               r["inv_perm"], None, None, None, None)
    tk_kernel.dispatch_mx_gather_scales(x_e8m0, r["perm"], top_k, r["offsets"], r["mtile_offsets"],
                                        rows, r["xw"])
    tk_kernel.dispatch_grouped_gemm1_mx(x_q, r["xw"], r["perm"], top_k, w13_q, w13_words, r["offsets"],
                                        r["mtile_offsets"], r["hq"], r["hw"], r["tile_ctr"][:8],
                                        packed=packed, mtile_list=r["mtile_list"])
    if keep_h:  # static tile order for the inspection pass
        r["h"] = torch.empty((rows, inter), dtype=torch.bfloat16, device=dev)
        tk_kernel.dispatch_grouped_gemm1_mx(x_q, r["xw"], r["perm"], top_k, w13_q, w13_words,
                                            r["offsets"], r["mtile_offsets"], r["h"], None, packed=packed)
    tk_kernel.dispatch_grouped_gemm2_mx(r["hq"], r["hw"], w2_q, w2_words, r["offsets"], r["mtile_offsets"],
                                        r["y"], r["tile_ctr"][8:], packed=packed, mtile_list=r["mtile_list"])
    tk_kernel.dispatch_combine(r["y"], r["topk_w"], r["inv_perm"], r["out"])
    return r


class MoELayerMX:
    """MX FP8 MoE FFN layer: e4m3 expert weights with 1x32 e8m0 exponents
    (uint8 [E, 2I, H/32] and [E, H, I/32]); activations come with their e8m0
    exponents [T, H/32] (see :func:`quant_mx`).  Weights and their exponents
    are packed once, here; each call is one hkmoe_moe_forward_mx."""

    def __init__(self, w13_q, w13_e8m0, w2_q, w2_e8m0, top_k, pack=True):
        _check_dev(w13_q, w2_q, w13_e8m0, w2_e8m0)
        if w13_q.dtype != F8 or w2_q.dtype != F8:
            raise RuntimeError("MoELayerMX: weights must be float8_e4m3fn")
        if w13_e8m0.dtype != torch.uint8 or w2_e8m0.dtype != torch.uint8:
            raise RuntimeError("MoELayerMX: weight exponents must be uint8 e8m0")
        self.packed = bool(pack)
        if self.packed:
            self.w13_q, self.w2_q = pack_weights(w13_q, gate_up=True), pack_weights(w2_q)
        else:
            self.w13_q, self.w2_q = w13_q.contiguous(), w2_q.contiguous()
        self.w13_words = mx_pack_weight_scales(w13_e8m0, gate_up=True)
        self.w2_words = mx_pack_weight_scales(w2_e8m0)
        self.top_k = int(top_k)
        self.num_experts, two_i, self.hidden = w13_q.shape
        self.inter = two_i // 2
        self._ws = None

    def workspace(self, num_tokens, device):
        need = tk_kernel.moe_workspace_size(num_tokens, self.num_experts, self.top_k, self.hidden,
                                            self.inter, tk_kernel.SCALE_MX)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=device)
        return self._ws

    def __call__(self, x_q, x_e8m0, logits, out=None):
        t = x_q.shape[0]
        if out is None:
            out = torch.empty((t, self.hidden), dtype=torch.bfloat16, device=x_q.device)
        tk_kernel.dispatch_moe_mx(x_q, x_e8m0, logits, self.w13_q, self.w13_words, self.w2_q, self.w2_words,
                                  self.top_k, out, self.workspace(t, x_q.device), packed=self.packed)
        return out
