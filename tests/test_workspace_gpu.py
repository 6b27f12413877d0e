"""Workspace sharing and stream placement of the kernels that use scratch.

Every plan's workspace starts with the W8A8 decode kernel's arrival counters
(64 KiB); the MX x bf16 upcast writes only after them.  So one workspace,
zeroed once, serves an upcast launch and a decode launch in either order
(tx_dot_launch through the C-ABI, one buffer for both).  And the Python
binding allocates and zero-fills a stream's workspace on that stream, so
dot() and dot_scaled() on a side stream see zeroed counters.  Decode outputs
are checked against the oracle bit for bit (int32 exact); the upcast dot
against the same dot on a fresh workspace, bit for bit.
"""
import ctypes

import numpy as np
import pytest

import oracle
import triton_ext_amd as tx
from dotcase import from_device, say, to_device, uniform_i8, uniform_scales
from test_mx_gpu import FMT, mx_bf16_case

pytestmark = pytest.mark.gpu


def _launch(plan, a, b, c, sa, sb, ws, stream):
    L = tx.load()
    rc = L.tx_dot_launch(ctypes.byref(plan), a.data_ptr(), b.data_ptr(), c.data_ptr(),
                         None if sa is None else sa.data_ptr(),
                         None if sb is None else sb.data_ptr(),
                         ws.data_ptr(), ws.numel(), stream)
    assert rc == tx.OK, L.tx_get_last_error().decode()


def _w8a8_case(M, N, K, seed):
    a = uniform_i8((M, K), seed)
    b = uniform_i8((K, N), seed + 1)
    sa = uniform_scales(M, seed + 2)
    sb = uniform_scales(N, seed + 3)
    want = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 256, 128),
                            scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb)
    return a, b, sa, sb, want


def _mx_case(gpu, M, N, K, seed):
    import torch
    cs = mx_bf16_case(M, N, K, "b", "e4m3", seed)
    a16 = to_device(cs["a16"].view(np.int16), gpu).view(torch.bfloat16)
    return a16, to_device(cs["b"], gpu), to_device(cs["s"], gpu)


def test_one_workspace_for_upcast_and_decode(gpu):
    """MX x bf16, then W8A8 split-K decode, then MX x bf16 again, all on one workspace."""
    import torch
    stream = torch.cuda.current_stream().cuda_stream
    M, N, K = 256, 512, 1024
    pm = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.F32, b_type=tx.F8E4M3,
                              scale_mode=tx.SCALE_MX32))
    dm, dn, dk = 16, 8192, 8192
    pd = tx.plan(tx.make_desc(dm, dn, dk, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL))
    assert pm.kernel == tx.KERNEL_GEMM_MX_BF16 and pd.kernel == tx.KERNEL_DECODE_I8
    assert pd.split_k > 1
    ws = torch.zeros(max(int(pm.workspace_bytes), int(pd.workspace_bytes)), dtype=torch.uint8,
                     device=gpu)
    a16, codes, scales = _mx_case(gpu, M, N, K, 71)
    c_ref = torch.empty((M, N), dtype=torch.float32, device=gpu)
    fresh = torch.zeros(int(pm.workspace_bytes), dtype=torch.uint8, device=gpu)
    _launch(pm, a16, codes, c_ref, None, scales, fresh, stream)
    a, b, sa, sb, want = _w8a8_case(dm, dn, dk, 72)
    da, db, dsa, dsb = (to_device(x, gpu) for x in (a, b, sa, sb))
    for rep in range(2):
        say(f"shared workspace: MX x bf16 {M}x{N}x{K}, then W8A8 {dm}x{dn}x{dk} (rep {rep})")
        c_mx = torch.full((M, N), float("nan"), dtype=torch.float32, device=gpu)
        _launch(pm, a16, codes, c_mx, None, scales, ws, stream)
        c_dec = torch.full((dm, dn), float("nan"), dtype=torch.bfloat16, device=gpu)
        _launch(pd, da, db, c_dec, dsa, dsb, ws, stream)
        torch.cuda.synchronize()
        assert torch.equal(c_mx.view(torch.int32), c_ref.view(torch.int32))
        got = from_device(c_dec)
        assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} outputs differ"
    # the counters are back at zero after the decode launches
    assert int(ws[:64 << 10].count_nonzero()) == 0


def test_side_stream_dot_and_dot_scaled(gpu):
    """dot() (W8A8 split-K decode) and dot_scaled() (MX x bf16) on a side stream, with the
    binding's workspace for that stream: results against the oracle."""
    import torch
    side = torch.cuda.Stream(device=gpu)  # default priority
    a, b, sa, sb, want = _w8a8_case(16, 8192, 8192, 81)
    M, N, K = 128, 256, 512
    a16, codes, scales = _mx_case(gpu, M, N, K, 82)
    with torch.cuda.stream(side):
        da, db, dsa, dsb = (to_device(x, gpu) for x in (a, b, sa, sb))
    side.synchronize()
    ref_mx = tx.dot_scaled(a16, None, "bf16", codes, scales, "e4m3")
    torch.cuda.synchronize()
    for rep in range(2):
        say(f"side stream: W8A8 16x8192x8192 and MX x bf16 {M}x{N}x{K} (rep {rep})")
        c = tx.dot(da, db, scale_a=dsa, scale_b=dsb, out_dtype=torch.bfloat16,
                   stream=side.cuda_stream)
        cm = tx.dot_scaled(a16, None, "bf16", codes, scales, "e4m3", stream=side.cuda_stream)
        side.synchronize()
        got = from_device(c)
        assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} outputs differ"
        assert torch.equal(cm.view(torch.int32), ref_mx.view(torch.int32))
