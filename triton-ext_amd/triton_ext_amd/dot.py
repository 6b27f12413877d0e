"""`dot()` over torch device tensors, through the tx_dot C-ABI.

torch provides the device memory and the current HIP stream; all arithmetic
runs in libmi355x_dot.so's kernels.
"""
import ctypes
import math

from . import capi

_TORCH_TYPES = {}
_workspaces = {}


def tx_type(t):
    import torch
    if not _TORCH_TYPES:
        _TORCH_TYPES.update({torch.float32: capi.F32, torch.float16: capi.F16,
                             torch.bfloat16: capi.BF16, torch.int8: capi.I8,
                             torch.float8_e4m3fn: capi.F8E4M3, torch.uint8: capi.F8E4M3,
                             torch.int32: capi.I32, torch.float8_e5m2: capi.F8E5M2})
    if t.dtype not in _TORCH_TYPES:
        raise TypeError(f"unsupported dtype {t.dtype}")
    return _TORCH_TYPES[t.dtype]


def _torch_dtype(tx):
    import torch
    return {capi.F32: torch.float32, capi.F16: torch.float16, capi.BF16: torch.bfloat16,
            capi.I32: torch.int32}[tx]


def _row_pitch(cols, elt_bytes):
    """Elements per row rounded up to a 16-byte multiple."""
    q = 16 // math.gcd(16, elt_bytes)
    return -(-cols // q) * q


def new_output(M, N, dtype, device):
    """An [M, N] tensor whose rows start 16 bytes apart as the kernels need:
    a view of [M, N'] storage, N' = N rounded up to whole 16-byte rows."""
    import torch
    elt = torch.empty(0, dtype=dtype).element_size()
    ld = _row_pitch(N, elt)
    return torch.empty((M, ld), dtype=dtype, device=device)[:, :N]


def _out_ldc(out):
    """C's row stride for a plan: out's own (which must start rows 16 bytes
    apart), or, for a single row, any 16-byte pitch (never used)."""
    if out.dim() != 2 or (out.shape[1] > 1 and out.stride(1) != 1):
        raise ValueError("out must be a row-major [M, N] tensor")
    if out.shape[0] <= 1:
        return _row_pitch(max(out.shape[1], 1), out.element_size())
    if (out.stride(0) * out.element_size()) % 16 or out.data_ptr() % 16:
        raise ValueError("out's rows must start 16 bytes apart on a 16-byte aligned base "
                         "(new_output makes such a tensor)")
    return out.stride(0)


def _layout(t, col_ok=True):
    """How a 2-D view lies in memory: ("row", row stride) when its rows are
    contiguous, ("col", column stride) when its columns are (a transposed
    view of row-major storage; only if col_ok), else (None, 0).  The stride
    of a dimension of size 1 says nothing about the layout: a single row
    whose elements lie apart is a transposed view, and a single column is
    row-major, or, when col_ok and its elements are adjacent, a transposed
    view (as a K-major B it then needs no copy)."""
    R, C = t.shape
    s0, s1 = t.stride()
    if col_ok and C <= 1 < R and s0 == 1 and s1 != 1:
        return "col", s1
    if C <= 1 or s1 == 1:
        return "row", s0
    if col_ok and (R <= 1 or s0 == 1):
        return "col", s1
    return None, 0


def _b_col_ok(b):
    """B may be K-major (a transposed view): 16-bit and 8-bit operands (every
    epilogue of dot(); tl.dot_scaled's MX operands take B as [K][N])."""
    return b.element_size() in (1, 2)


def _kmajor_plans(a, b, c_tx, scale_mode, block, flags):
    """Whether the planner takes this dot with B K-major: always with its own
    tile choice (block (0, 0, 0)), and for a block asked for when that tile has
    a K-major form (asked of the planner, on 16-byte strides)."""
    if tuple(block) == (0, 0, 0):
        return True
    M, K = a.shape
    N = b.shape[1]
    d = capi.make_desc(M, N, K, tx_type(a), c_tx, b_type=tx_type(b), scale_mode=scale_mode,
                       block=block, lda=_row_pitch(K, 1), ldb=_row_pitch(K, 1),
                       ldc=_row_pitch(N, 1), flags=flags | capi.FLAG_B_KMAJOR)
    p = capi.DotPlan()
    return capi.load().tx_dot_plan_create(ctypes.byref(d), ctypes.byref(p)) == capi.OK


def _b_kmajor_ok(a, b, c_tx, scale_mode, block, flags):
    return (a.dim() == 2 and b.dim() == 2 and _b_col_ok(b)
            and _kmajor_plans(a, b, c_tx, scale_mode, block, flags))


def aligned_rows(t, col_ok=True):
    """t itself when its rows (or, for a transposed view and col_ok, its
    columns) start 16 bytes apart on a 16-byte aligned base, else a copy in
    padded storage of the same layout (row-major when not col_ok).  The
    kernels read 16-byte chunks; K and N themselves may be any size."""
    import torch
    if t.dim() != 2 or t.numel() == 0:
        return t
    elt = t.element_size()
    kind, ld = _layout(t, col_ok)
    if kind is not None and (ld * elt) % 16 == 0 and t.data_ptr() % 16 == 0:
        return t
    if kind == "col":  # [N][K] storage viewed as [K][N]
        return aligned_rows(t.t().contiguous()).t()
    if kind is None or t.stride(1) != 1:
        t = t.contiguous()
    buf = torch.empty((t.shape[0], _row_pitch(t.shape[1], elt)), dtype=t.dtype, device=t.device)
    buf[:, :t.shape[1]].copy_(t)
    return buf[:, :t.shape[1]]


def plan_for(a, b, out_dtype_tx, scale_mode=capi.SCALE_NONE, block=(0, 0, 0), flags=0, ldc=0):
    """Plan C = A @ B.  B may be row-major [K,N] or a transposed view of a
    row-major [N,K] tensor (K-major, e.g. `k.t()` in q @ k.T).  ldc: C's row
    stride (0: packed)."""
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"dot of {tuple(a.shape)} and {tuple(b.shape)}")
    M, K = a.shape
    N = b.shape[1]
    a_kind, a_ld = _layout(a, col_ok=False)
    b_kind, b_ld = _layout(b, col_ok=_b_kmajor_ok(a, b, out_dtype_tx, scale_mode, block, flags))
    if a_kind == "row" and b_kind is None and _layout(b)[0] == "col":
        raise ValueError("B is a transposed view, and the tile asked for has no K-major "
                         "form; copy it row-major")
    if a_kind != "row" or b_kind is None:
        raise ValueError("A rows must be contiguous, and B rows (or B's columns) too")
    b_kmajor = b_kind == "col"
    if b_kmajor:
        flags |= capi.FLAG_B_KMAJOR
    # an empty operand's strides are arbitrary: describe it as packed
    lda = a_ld if M > 0 and K > 0 else 0
    ldb = b_ld if K > 0 and N > 0 else 0
    desc = capi.make_desc(M, N, K, tx_type(a), out_dtype_tx, b_type=tx_type(b),
                          scale_mode=scale_mode, block=block, lda=lda, ldb=ldb, ldc=ldc,
                          flags=flags)
    return capi.plan(desc)


def workspace_for(p, device, stream):
    """A zero-initialised workspace of at least p.workspace_bytes, cached per
    (device, stream): launches on one stream run one after another, so they
    may share it; launches on different streams may overlap and get their own.

    Every plan's workspace starts with the decode kernel's arrival counters,
    which must start at zero and which every completed launch leaves at zero
    (the MX upcast writes only after them), so one buffer serves every plan.
    The buffer is allocated and zero-filled on `stream` itself, so the fill
    runs before any launch enqueued there after it, and torch's caching
    allocator orders the release of a buffer that grew too small after that
    stream's queued work.
    """
    import torch
    if p.workspace_bytes == 0:
        return None
    key = (str(device), int(stream or 0))
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < p.workspace_bytes:
        s = (torch.cuda.ExternalStream(int(stream), device=device) if stream
             else torch.cuda.default_stream(device))
        with torch.cuda.device(device), torch.cuda.stream(s):
            ws = torch.zeros(int(p.workspace_bytes), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def dot(a, b, out=None, out_dtype=None, scale_a=None, scale_b=None, scale_mode=None,
        block=(0, 0, 0), flags=0, plan=None, workspace=None, stream=None, acc=None):
    """C = epilogue(A @ B) on the current device's stream.

    scale_mode defaults to ROWCOL when int8 operands come with scales, to
    BLOCK128 for fp8 operands with scales, else NONE.  acc (fp32 or int32
    [M, N]): returns acc + A @ B, as tl.dot(a, b, acc) does, in a new tensor
    (or in `out`); the kernel adds its finished sum to C.

    K and N may be any size.  Operands whose rows do not start 16 bytes
    apart are copied to padded storage first (one extra pass), as is a
    transposed view of A in row-major form (a transposed B runs K-major,
    unless `block` names a tile without that form: then B is copied too); a
    new output is a view of padded storage; a given `out` must already have
    16-byte row strides.
    """
    import torch
    ta = tx_type(a)
    if scale_mode is None:
        if scale_a is None:
            scale_mode = capi.SCALE_NONE
        else:
            scale_mode = capi.SCALE_ROWCOL if ta == capi.I8 else capi.SCALE_BLOCK128
    if out is not None:
        c_tx = tx_type(out)
    elif acc is not None and acc.dtype in (torch.float32, torch.int32):
        c_tx = tx_type(acc)  # the new output is a copy of acc
    elif out_dtype is not None:
        c_tx = tx_type(torch.empty(0, dtype=out_dtype))
    else:
        c_tx = capi.I32 if (ta == capi.I8 and scale_mode == capi.SCALE_NONE) else (
            capi.BF16 if ta in (capi.BF16, capi.I8, capi.F8E4M3) else capi.F32)
    if acc is not None:
        flags |= capi.FLAG_ACCUMULATE
    if plan is None:
        a = aligned_rows(a, col_ok=False)
        b = aligned_rows(b, col_ok=_b_kmajor_ok(a, b, c_tx, scale_mode, block, flags))
    if acc is not None:
        if acc.dtype not in (torch.float32, torch.int32) or acc.dim() != 2:
            raise ValueError("acc must be an fp32 or int32 [M, N] tensor")
        if out is None:
            out = new_output(acc.shape[0], acc.shape[1], acc.dtype, acc.device)
            out.copy_(acc)
        elif out.data_ptr() != acc.data_ptr():
            out.copy_(acc)
    M, N = a.shape[0], b.shape[1]
    if out is None:
        out = new_output(M, N, _torch_dtype(c_tx), a.device)
    ldc = _out_ldc(out)
    p = plan if plan is not None else plan_for(a, b, c_tx, scale_mode, block, flags, ldc=ldc)
    if bool(p.desc.flags & capi.FLAG_ACCUMULATE) != (acc is not None):
        raise ValueError("plan and call disagree on acc: the plan's FLAG_ACCUMULATE must be "
                         "set exactly when acc is given")
    if M > 1 and ldc != p.desc.ldc:
        raise ValueError(f"out's row stride {ldc} differs from the plan's ldc {p.desc.ldc}")
    if stream is None:
        stream = torch.cuda.current_stream(a.device).cuda_stream
    ws = workspace if workspace is not None else workspace_for(p, a.device, stream)
    L = capi.load()
    capi.check(L.tx_dot_launch(ctypes.byref(p), a.data_ptr(), b.data_ptr(), out.data_ptr(),
                               None if scale_a is None else scale_a.data_ptr(),
                               None if scale_b is None else scale_b.data_ptr(),
                               None if ws is None else ws.data_ptr(),
                               0 if ws is None else ws.numel(), stream))
    return out


_MX_FORMATS = {"e4m3": capi.F8E4M3, "e5m2": capi.F8E5M2, "e2m1": capi.F4E2M1}


def dot_scaled(lhs, lhs_scale, lhs_format, rhs, rhs_scale, rhs_format, acc=None,
               fast_math=False, lhs_k_pack=True, rhs_k_pack=True, out_dtype=None, out=None,
               block=(0, 0, 0), plan=None, stream=None):
    """tl.dot_scaled over torch device tensors (T:language/core.py:2064-2101).

    lhs [M, K] (e2m1: uint8 [M, K/2], two elements per byte, even K in the
    low nibble), rhs [K, N] (e2m1: uint8 [K/2, N]); fp8 operands as
    float8_e4m3fn / float8_e5m2 or their uint8 bits.  lhs_scale uint8
    [M, K/32] and rhs_scale uint8 [N, K/32] hold e8m0 exponents (2^(s-127)),
    rhs_scale indexed by column first and not transposed.  Returns fp32 (or
    bf16 with out_dtype=torch.bfloat16) [M, N].  A scale of None leaves that
    operand unscaled (T:language/semantic.py:1625-1626): it runs as e8m0 127
    (2^0), which is exact.  One operand may be "bf16" (a torch.bfloat16
    tensor, no scale): the other is upcast to bf16 and a bf16 dot runs, as
    tl.dot_scaled specifies (T:language/core.py:2072-2076).  Checks follow
    T:language/semantic.py:1597-1665; what this backend does not implement
    (fp16 operands, bf16 on both sides, e2m1 mixed with fp8, packing along M
    or N) raises NotImplementedError.  acc (fp32 [M, N]) returns acc + the
    dot, as tl.dot_scaled's acc does.  Scales given as torch.float8_e4m3fn
    are e4m3 multipliers per 16 K ([M, K/16], [N, K/16]; Triton's fp8e4nv
    scales): e2m1 (or bf16) operands, run through a bf16 upcast.  As in
    dot(), operands whose rows do not start 16 bytes apart are copied to
    padded storage first.
    """
    import torch
    for name, fmt in (("lhs_format", lhs_format), ("rhs_format", rhs_format)):
        if fmt not in ("e2m1", "e4m3", "e5m2", "bf16", "fp16"):
            raise ValueError(f"NYI: {name} {fmt}")
        if fmt not in _MX_FORMATS and fmt != "bf16":
            raise NotImplementedError(f"{name} {fmt}: e4m3, e5m2, e2m1 and bf16 are implemented")
    if lhs_format == "bf16" and rhs_format == "bf16":
        raise NotImplementedError("bf16 on both sides is tl.dot, not dot_scaled")
    for fmt, t, sc, nm in ((lhs_format, lhs, lhs_scale, "lhs"), (rhs_format, rhs, rhs_scale, "rhs")):
        if fmt == "bf16" and (t.dtype != torch.bfloat16 or sc is not None):
            raise ValueError(f"{nm}: a bf16 operand is a torch.bfloat16 tensor with no scale")
    if acc is not None:
        if acc.dtype != torch.float32 or (out_dtype not in (None, torch.float32)):
            raise ValueError("acc must be fp32, as tl.dot_scaled's out_dtype")
    if not lhs_k_pack or not rhs_k_pack:
        raise NotImplementedError("only K-packed e2m1 operands are implemented")
    if lhs.dim() != 2 or rhs.dim() != 2:
        raise ValueError(f"Both inputs must be 2D; (lhs: {tuple(lhs.shape)} vs rhs: "
                         f"{tuple(rhs.shape)})")
    pa = 2 if lhs_format == "e2m1" else 1
    pb = 2 if rhs_format == "e2m1" else 1
    M, K = lhs.shape[0], lhs.shape[1] * pa
    N = rhs.shape[1]
    if rhs.shape[0] * pb != K:
        raise ValueError("Reduction dimension should pack the same number of elements; "
                         f"(lhs: {tuple(lhs.shape)} vs rhs: {tuple(rhs.shape)})")
    # e4m3 scales: one per 16 K (T:language/semantic.py:1597-1609)
    nv = any(t is not None and t.dtype == torch.float8_e4m3fn for t in (lhs_scale, rhs_scale))
    if nv and (lhs_format not in ("e2m1", "bf16") or rhs_format not in ("e2m1", "bf16")):
        raise NotImplementedError("e4m3 scales are implemented for e2m1 operands")
    g = 16 if nv else 32
    # scale None: the operand is unscaled -- e8m0 127 (2^0), or e4m3 1.0
    # (0x38) -- in every group (a bf16 operand has none and reads none)
    unit = 0x38 if nv else 127
    if lhs_scale is None and lhs_format != "bf16":
        lhs_scale = torch.full((M, K // g), unit, dtype=torch.uint8, device=lhs.device)
    if rhs_scale is None and rhs_format != "bf16":
        rhs_scale = torch.full((N, K // g), unit, dtype=torch.uint8, device=rhs.device)
    if nv:
        lhs_scale, rhs_scale = (t.view(torch.uint8) if t is not None and t.dtype != torch.uint8
                                else t for t in (lhs_scale, rhs_scale))
    if lhs_scale is not None and tuple(lhs_scale.shape) != (M, K // g):
        raise ValueError(f"lhs_scale must be a tensor of shape [{M}, {K // g}]. "
                         f"Got {list(lhs_scale.shape)}")
    if rhs_scale is not None and tuple(rhs_scale.shape) != (N, K // g):
        raise ValueError(f"rhs_scale must be a tensor of shape [{N}, {K // g}]. "
                         f"Got {list(rhs_scale.shape)}")
    for t, nm in ((lhs_scale, "lhs_scale"), (rhs_scale, "rhs_scale")):
        if t is not None and (t.dtype != torch.uint8 or not t.is_contiguous()):
            raise ValueError(f"{nm} must be a contiguous uint8 (e8m0) or float8_e4m3fn tensor")
    if _layout(lhs, False)[0] != "row" or _layout(rhs, False)[0] != "row":
        raise ValueError("lhs and rhs rows must be contiguous")
    if plan is None:
        lhs, rhs = aligned_rows(lhs, col_ok=False), aligned_rows(rhs, col_ok=False)
    flags = 0
    if acc is not None:  # acc + dot, in a new tensor (or `out`), as tl.dot_scaled(acc=)
        if out is None:
            out = new_output(acc.shape[0], acc.shape[1], acc.dtype, acc.device)
            out.copy_(acc)
        elif out.data_ptr() != acc.data_ptr():
            out.copy_(acc)
        flags = capi.FLAG_ACCUMULATE
    if out is not None:
        c_tx = tx_type(out)
    else:
        c_tx = capi.BF16 if out_dtype == torch.bfloat16 else capi.F32
    if out is None:
        out = new_output(M, N, _torch_dtype(c_tx), lhs.device)
    ldc = _out_ldc(out)
    if plan is None:
        lda = lhs.stride(0) * pa if M > 0 and K > 0 else 0
        ldb = rhs.stride(0) if K > 0 and N > 0 else 0
        desc = capi.make_desc(M, N, K, _MX_FORMATS.get(lhs_format, capi.BF16), c_tx,
                              b_type=_MX_FORMATS.get(rhs_format, capi.BF16),
                              scale_mode=capi.SCALE_NV16 if nv else capi.SCALE_MX32,
                              block=block, lda=lda, ldb=ldb, ldc=ldc, flags=flags)
        plan = capi.plan(desc)
    elif bool(plan.desc.flags & capi.FLAG_ACCUMULATE) != (acc is not None):
        raise ValueError("plan and call disagree on acc: the plan's FLAG_ACCUMULATE must be "
                         "set exactly when acc is given")
    if M > 1 and ldc != plan.desc.ldc:
        raise ValueError(f"out's row stride {ldc} differs from the plan's ldc {plan.desc.ldc}")
    if stream is None:
        stream = torch.cuda.current_stream(lhs.device).cuda_stream
    ws = workspace_for(plan, lhs.device, stream)
    L = capi.load()
    capi.check(L.tx_dot_launch(ctypes.byref(plan), lhs.data_ptr(), rhs.data_ptr(),
                               out.data_ptr(),
                               None if lhs_scale is None else lhs_scale.data_ptr(),
                               None if rhs_scale is None else rhs_scale.data_ptr(),
                               None if ws is None else ws.data_ptr(),
                               0 if ws is None else ws.numel(), stream))
    return out


def attention(q, k, v, causal, sm_scale, USE_TMA=True, *, return_lse=False, plan=None,
              stream=None, block=(0, 0)):
    """Forward of the fused-attention tutorial's `attention(q, k, v, causal,
    sm_scale, USE_TMA=True)` (R:pass/LoopSplit/06-fused-attention.py:583-640) on the
    MI355X kernel: q, k, v [Z, H, N_CTX, HEAD_DIM], head dim 16, 32, 64, 128
    or 256, in fp16 or bf16 (head dim contiguous) or in float8_e5m2 as the
    tutorial's fp8 provider passes them (:774-779): q and k head-dim contiguous, v
    key-contiguous (stride 1 along N_CTX, "when v is in float8_e5m2 it is
    transposed", :586).  o has q's type; p is rounded to it before p @ v
    (:81-84).  Returns o (and M, the base-2 logsumexp [Z, H, N_CTX] the
    tutorial saves for its backward, with return_lse=True).  Shape checks
    follow the tutorial's asserts.  block = (BLOCK_M, BLOCK_N), one of the
    tutorial's autotuned configs (:145-159): BLOCK_M 64 or 128 by BLOCK_N 32
    or 64 (not 128 x 32 at head dims below 64, or below 128 in fp8); (0, 0)
    takes 128 x 64.  USE_TMA is accepted for the
    tutorial's signature and has no effect (gfx950 has no tensor memory
    accelerator; the tutorial's HIP path takes the pointer kernel too).
    return_lse, plan, stream and block are keyword-only.
    """
    import torch
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must share one [Z, H, N_CTX, HEAD_DIM] shape: "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    HEAD_DIM = q.shape[-1]
    if HEAD_DIM not in {16, 32, 64, 128, 256}:
        raise ValueError(f"HEAD_DIM {HEAD_DIM} not in {{16, 32, 64, 128, 256}}")
    fp8 = q.dtype == torch.float8_e5m2
    if q.dtype not in (torch.float16, torch.bfloat16) and not fp8:
        raise NotImplementedError(f"q: fp16, bf16 and float8_e5m2 are implemented, got {q.dtype}")
    for t, nm in ((k, "k"), (v, "v")):
        if t.dtype != q.dtype:
            raise ValueError(f"{nm} is {t.dtype}, q is {q.dtype}")
    for t, nm in ((q, "q"), (k, "k")) + ((() if fp8 else ((v, "v"),))):
        if t.stride(3) != 1:
            raise ValueError(f"{nm}: the head dimension must be contiguous")
    if fp8 and v.stride(2) != 1:
        raise ValueError("v: float8_e5m2 v must be key-contiguous (stride 1 along N_CTX), "
                         "as v.permute(0, 1, 3, 2).contiguous().permute(0, 1, 3, 2) makes it")
    Z, H, N = q.shape[:3]
    o = torch.empty_like(q, memory_format=torch.contiguous_format)
    M = torch.empty((Z, H, N), device=q.device, dtype=torch.float32)
    if plan is None:
        st = {nm: (t.stride(0), t.stride(1), t.stride(2)) for nm, t in
              (("q", q), ("k", k), ("v", v), ("o", o))}
        if fp8:
            st["v"] = (v.stride(0), v.stride(1), v.stride(3))  # dim rows of N_CTX keys
        dt = capi.F8E5M2 if fp8 else capi.BF16 if q.dtype == torch.bfloat16 else capi.F16
        plan = capi.attn_plan(Z, H, N, HEAD_DIM, causal, sm_scale, dtype=dt, strides=st,
                              block=block)
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    capi.check(capi.load().tx_attn_fwd_launch(ctypes.byref(plan), q.data_ptr(), k.data_ptr(),
                                              v.data_ptr(), o.data_ptr(), M.data_ptr(), stream))
    return (o, M) if return_lse else o
