"""Seeded fuzz of the planners and the launch-time plan check, through the C-ABI
(no GPU: a launch that passes every check stops at TX_ERR_NO_DEVICE).

Properties:
  * tx_dot_plan_create / tx_attn_fwd_plan answer every descriptor -- valid,
    edge-sized or adversarial -- with TX_OK, TX_ERR_INVALID or
    TX_ERR_UNSUPPORTED (the reference's return-code convention,
    R:infra/pass/TritonExtPassInfra.cpp:22-23), never a crash;
  * an accepted dot plan satisfies what its kernel assumes: the loop split
    (R:pass/LoopSplit/LoopSplit.cpp:156-174), the tile grid, and operand spans
    below 2 GiB on the 32-bit-offset tiles;
  * every plan the planner makes passes the launch's own check (the launch
    gets as far as looking for the device);
  * a plan with one launch-relevant field changed is refused at launch with
    TX_ERR_INVALID or TX_ERR_UNSUPPORTED, before any HIP call.
"""
import ctypes
import os

import numpy as np
import pytest

import triton_ext_amd as tx
from triton_ext_amd import capi

# TX_FUZZ_SEED draws other descriptors (the committed set is the default)
SEED = int(os.environ.get("TX_FUZZ_SEED", "424242"))
OKS = {tx.OK, tx.ERR_INVALID, tx.ERR_UNSUPPORTED}

# (a_type, b_type, c_type, scale_mode): every operand form the planner knows,
# and a few it must refuse
FORMS = [
    (tx.BF16, tx.BF16, tx.BF16, tx.SCALE_NONE), (tx.BF16, tx.BF16, tx.F32, tx.SCALE_NONE),
    (tx.F16, tx.F16, tx.F16, tx.SCALE_NONE), (tx.F16, tx.F16, tx.F32, tx.SCALE_NONE),
    (tx.I8, tx.I8, tx.I32, tx.SCALE_NONE), (tx.I8, tx.I8, tx.BF16, tx.SCALE_ROWCOL),
    (tx.F8E4M3, tx.F8E4M3, tx.BF16, tx.SCALE_BLOCK128),
    (tx.F8E4M3, tx.F8E4M3, tx.F32, tx.SCALE_BLOCK128),
    (tx.F8E4M3, tx.F8E4M3, tx.F32, tx.SCALE_NONE), (tx.F8E5M2, tx.F8E5M2, tx.F32, tx.SCALE_NONE),
    (tx.F8E4M3, tx.F8E5M2, tx.F32, tx.SCALE_NONE),
    (tx.F8E4M3, tx.F8E4M3, tx.F32, tx.SCALE_MX32), (tx.F8E5M2, tx.F8E4M3, tx.BF16, tx.SCALE_MX32),
    (tx.F4E2M1, tx.F4E2M1, tx.F32, tx.SCALE_MX32), (tx.BF16, tx.F8E4M3, tx.F32, tx.SCALE_MX32),
    (tx.F4E2M1, tx.BF16, tx.BF16, tx.SCALE_MX32), (tx.F4E2M1, tx.F4E2M1, tx.F32, tx.SCALE_NV16),
    (tx.BF16, tx.F4E2M1, tx.F32, tx.SCALE_NV16),
    # refused forms
    (tx.F32, tx.F32, tx.F32, tx.SCALE_NONE), (tx.BF16, tx.F16, tx.F32, tx.SCALE_NONE),
    (tx.I8, tx.I8, tx.F32, tx.SCALE_NONE), (tx.F8E4M3, tx.F8E4M3, tx.BF16, tx.SCALE_NONE),
]
BITS = {tx.F32: 32, tx.F16: 16, tx.BF16: 16, tx.I8: 8, tx.F8E4M3: 8, tx.I32: 32, tx.F8E5M2: 8,
        tx.F4E2M1: 4}
BLOCKS = [(0, 0, 0)] * 6 + [(256, 256, 64), (128, 128, 64), (64, 64, 32), (256, 256, 128),
                            (256, 224, 128), (128, 128, 128), (96, 64, 64), (-1, 0, 0)]


def _dim(rng):
    r = rng.random()
    if r < 0.04:
        return 0
    if r < 0.08:
        return int(rng.choice([-1, 1 << 31, (1 << 31) - 1, 70000, 65536 * 3]))
    if r < 0.35:
        return int(rng.integers(1, 40))
    if r < 0.8:
        return int(rng.choice([16, 32, 64, 128, 256, 4096, 8192])) + int(rng.integers(-3, 4))
    return int(rng.integers(1, 20000))


def _stride(rng, cols, bits):
    """0 (packed), the row padded to 16 bytes, an unaligned one, or a short one."""
    r = rng.random()
    if r < 0.15 or cols <= 0:
        return 0
    q = max(1, 128 // bits)  # elements per 16 bytes
    if r < 0.9:
        return -(-cols // q) * q + q * int(rng.integers(0, 3))
    if r < 0.95:
        return cols + 1
    return max(1, cols - 1)


def _random_desc(rng):
    a, b, c, sm = FORMS[int(rng.integers(len(FORMS)))]
    M, N, K = _dim(rng), _dim(rng), _dim(rng)
    flags = 0
    if a in (tx.BF16, tx.F16) and b == a and rng.random() < 0.25:
        flags |= tx.FLAG_B_KMAJOR
    if c in (tx.F32, tx.I32) and rng.random() < 0.2:
        flags |= tx.FLAG_ACCUMULATE
    if rng.random() < 0.05:
        flags |= 1  # TX_FLAG_NO_LOOP_SPLIT
    if rng.random() < 0.02:
        flags |= 1 << 7  # unknown
    kmajor = bool(flags & tx.FLAG_B_KMAJOR)
    lda = _stride(rng, K, BITS.get(a, 8))
    ldb = _stride(rng, K if kmajor else N, BITS.get(b, 8))
    ldc = _stride(rng, N, BITS.get(c, 8))
    blk = BLOCKS[int(rng.integers(len(BLOCKS)))]
    return tx.make_desc(M, N, K, a, c, b_type=b, scale_mode=sm, block=blk, lda=lda, ldb=ldb,
                        ldc=ldc, flags=flags)


def _spans(d):
    """A's and B's byte spans as the tiles read them (e2m1 A: lda counts elements)."""
    ba, bb = BITS[d.a_type], BITS[d.b_type]
    kmajor = bool(d.flags & tx.FLAG_B_KMAJOR)
    if d.a_type == tx.F4E2M1:
        sa = (d.M - 1) * (d.lda // 2) + (d.K + 1) // 2
    else:
        sa = ((d.M - 1) * d.lda + d.K) * ba // 8
    if d.b_type == tx.F4E2M1:
        sb = ((d.K + 1) // 2 - 1) * d.ldb + d.N
    elif kmajor:
        sb = ((d.N - 1) * d.ldb + d.K) * bb // 8
    else:
        sb = ((d.K - 1) * d.ldb + d.N) * bb // 8
    return sa, sb


_BUF = ctypes.create_string_buffer(4096)
_ADDR = (ctypes.addressof(_BUF) + 255) & ~255  # 256-byte aligned host bytes


def _launch(p):
    """tx_dot_launch with aligned dummy pointers (never dereferenced on the host)."""
    L = capi.load()
    a = ctypes.c_void_p(_ADDR)
    return L.tx_dot_launch(ctypes.byref(p), a, a, a, a, a, a, 4096, None)


def _no_device():
    import torch
    return not torch.cuda.is_available()


def test_dot_planner_fuzz():
    L = capi.load()
    rng = np.random.default_rng(SEED)
    seen = {}
    for _ in range(6000):
        d = _random_desc(rng)
        p = capi.DotPlan()
        rc = L.tx_dot_plan_create(ctypes.byref(d), ctypes.byref(p))
        assert rc in OKS, (rc, L.tx_get_last_error())
        seen[rc] = seen.get(rc, 0) + 1
        if rc != tx.OK:
            assert L.tx_get_last_error(), "a refusal names its reason"
            continue
        q = p.desc
        assert (q.M, q.N, q.K, q.a_type, q.b_type, q.c_type) == (d.M, d.N, d.K, d.a_type,
                                                                   d.b_type, d.c_type)
        assert q.lda > 0 or q.K == 0 or q.M == 0
        bk, bm, bn = q.block_k, q.block_m, q.block_n
        assert bm > 0 and bn > 0 and bk > 0
        if q.flags & 1:
            assert (p.k_split, p.k_main_steps, p.k_tail) == (0, 0, q.K)
        else:
            assert p.k_split == q.K - (q.K % bk if q.K % bk else 0) or p.k_split == q.K
            assert p.k_split % bk == 0 and p.k_main_steps == p.k_split // bk
            assert p.k_tail == q.K - p.k_split and 0 <= p.k_tail < bk
        assert p.m_tiles == -(-q.M // bm) and p.n_tiles == -(-q.N // bn)
        assert p.m_edge == q.M % bm and p.n_edge == q.N % bn
        assert p.block_threads % 64 == 0 and 64 <= p.block_threads <= 1024
        assert p.workspace_bytes >= 0
        if p.kernel != tx.KERNEL_DECODE_I8 and (bm, bn) in ((256, 256), (256, 224)) \
                and p.kernel != tx.KERNEL_GEMM_MX_BF16:
            sa, sb = _spans(q)
            assert sa < 1 << 31 and sb < 1 << 31, "a 32-bit-offset tile past 2 GiB"
        if _no_device():
            rc2 = _launch(p)
            want = tx.OK if q.M == 0 or q.N == 0 else tx.ERR_NO_DEVICE
            assert rc2 == want, (rc2, L.tx_get_last_error(), q.M, q.N, q.K)
    # the fuzz reaches both sides
    assert seen.get(tx.OK, 0) > 600 and seen.get(tx.ERR_INVALID, 0) > 300 and \
        seen.get(tx.ERR_UNSUPPORTED, 0) > 300, seen


# Fields of a dot plan the kernels trust, with a change that must be refused.
TAMPER = [
    ("grid_x", lambda p: setattr(p, "grid_x", p.grid_x + 1)),
    ("block_threads", lambda p: setattr(p, "block_threads", p.block_threads * 2)),
    ("kernel", lambda p: setattr(p, "kernel", p.kernel % 8 + 1)),
    ("split_k", lambda p: setattr(p, "split_k", p.split_k * 2)),
    ("k_split", lambda p: setattr(p, "k_split", p.k_split + p.desc.block_k)),
    ("k_main_steps", lambda p: setattr(p, "k_main_steps", p.k_main_steps + 1)),
    ("k_tail", lambda p: setattr(p, "k_tail", p.k_tail + 1)),
    ("m_tiles", lambda p: setattr(p, "m_tiles", p.m_tiles + 1)),
    ("n_tiles", lambda p: setattr(p, "n_tiles", p.n_tiles - 1)),
    ("workspace_bytes", lambda p: setattr(p, "workspace_bytes", p.workspace_bytes + 16)),
    ("desc.M", lambda p: setattr(p.desc, "M", p.desc.M + p.desc.block_m)),
    ("desc.N", lambda p: setattr(p.desc, "N", p.desc.N + 1)),
    ("desc.lda", lambda p: setattr(p.desc, "lda", 0)),
    ("desc.ldb", lambda p: setattr(p.desc, "ldb", p.desc.ldb + 1)),
    ("desc.block_m", lambda p: setattr(p.desc, "block_m", p.desc.block_m * 2)),
    ("desc.block_k", lambda p: setattr(p.desc, "block_k", p.desc.block_k // 2)),
    ("desc.c_type", lambda p: setattr(p.desc, "c_type", tx.I32 if p.desc.c_type != tx.I32
                                      else tx.F32)),
    ("desc.flags", lambda p: setattr(p.desc, "flags", p.desc.flags ^ tx.FLAG_ACCUMULATE)),
]


@pytest.mark.parametrize("shape", [(300, 272, 416, tx.BF16, tx.F32, tx.SCALE_NONE),
                                   (4096, 4096, 4000, tx.BF16, tx.BF16, tx.SCALE_NONE),
                                   (512, 512, 512, tx.F16, tx.F32, tx.SCALE_NONE),
                                   (16, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL),
                                   (300, 304, 256, tx.I8, tx.I32, tx.SCALE_NONE),
                                   (2048, 7168, 7168, tx.F8E4M3, tx.BF16, tx.SCALE_BLOCK128),
                                   (512, 512, 1024, tx.F8E4M3, tx.F32, tx.SCALE_MX32)])
def test_tampered_dot_plans_are_refused_at_launch(shape):
    if not _no_device():
        pytest.skip("a visible GPU would take the launch past the checks")
    L = capi.load()
    M, N, K, a, c, sm = shape
    base = tx.plan(tx.make_desc(M, N, K, a, c, scale_mode=sm))
    assert _launch(base) == tx.ERR_NO_DEVICE, L.tx_get_last_error()
    for name, change in TAMPER:
        p = capi.DotPlan()
        ctypes.memmove(ctypes.byref(p), ctypes.byref(base), ctypes.sizeof(p))
        change(p)
        if bytes(p) == bytes(base):
            continue
        rc = _launch(p)
        if name == "desc.flags" and c in (tx.F32, tx.I32):
            # accumulating into an fp32 / int32 C is the same plan with the flag: consistent
            assert rc in (tx.ERR_NO_DEVICE, tx.ERR_INVALID), name
            continue
        assert rc in (tx.ERR_INVALID, tx.ERR_UNSUPPORTED), \
            f"{name}: launch answered {rc} ({L.tx_get_last_error()})"


def test_upcast_b_span_uses_the_upcast_row_stride():
    """MX x bf16 with ragged N near 2 GiB: the planner prices the upcast B at its real row
    stride (N rounded up to 16 columns, the stride the launch uses), so it picks a tile
    whose 32-bit offsets reach it -- the 128x128 tile here -- instead of a 256-wide tile
    that plan creation then refuses."""
    M, N, K = 3840, 3841, 278464
    p = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.F32, b_type=tx.F8E4M3, ldb=3856, ldc=3844,
                             scale_mode=tx.SCALE_MX32))
    assert p.kernel == tx.KERNEL_GEMM_MX_BF16
    assert (p.desc.block_m, p.desc.block_n) == (128, 128)
    # the upcast B: K rows of N rounded up to 16 bf16 columns, at or past 2^31 bytes
    assert (K - 1) * ((N + 15) // 16 * 16) * 2 + N * 2 >= 1 << 31
    if _no_device():  # the launch's own checks accept it (dummy pointers: never on a GPU)
        assert _launch(p) == tx.ERR_NO_DEVICE, capi.load().tx_get_last_error()


def test_attention_planner_fuzz_and_tampering():
    L = capi.load()
    rng = np.random.default_rng(SEED + 1)
    a = ctypes.c_void_p(_ADDR)
    accepted = 0
    for _ in range(3000):
        dt = int(rng.choice([tx.F16, tx.BF16, tx.F8E5M2, tx.F32]))
        hd = int(rng.choice([8, 16, 32, 48, 64, 128, 256]))
        bm, bn = [(0, 0), (64, 32), (64, 64), (128, 32), (128, 64), (256, 64), (64, 16)][
            int(rng.integers(7))]
        N = int(rng.choice([0, 64, 128, 192, 200, 256, 1024])) * int(rng.integers(1, 3))
        d = capi.AttnDesc()
        d.Z, d.H, d.N_CTX = int(rng.integers(-1, 4)), int(rng.integers(0, 5)), N
        d.head_dim, d.dtype, d.causal = hd, dt, int(rng.integers(0, 3))
        d.sm_scale = float(rng.choice([0.5, 1.3, float("nan"), float("inf")]))
        d.block_m, d.block_n = bm, bn
        if rng.random() < 0.2:  # a stride that is too short or unaligned
            d.q_sm = int(rng.choice([hd - 1, hd + 1, hd + 8]))
        p = capi.AttnPlan()
        rc = L.tx_attn_fwd_plan(ctypes.byref(d), ctypes.byref(p))
        assert rc in OKS, (rc, L.tx_get_last_error())
        if rc != tx.OK:
            continue
        accepted += 1
        assert p.grid_x == d.Z * d.H * (d.N_CTX // p.desc.block_m)
        assert p.block_threads == p.desc.block_m // 32 * 64
        if not _no_device():
            continue
        launch = lambda pl: L.tx_attn_fwd_launch(ctypes.byref(pl), a, a, a, a, a, None)
        want = tx.OK if p.grid_x == 0 else tx.ERR_NO_DEVICE
        assert launch(p) == want, L.tx_get_last_error()
        if p.grid_x == 0:
            continue
        for field, delta in (("grid_x", 1), ("block_threads", 64), ("m_blocks", 1)):
            t = capi.AttnPlan()
            ctypes.memmove(ctypes.byref(t), ctypes.byref(p), ctypes.sizeof(t))
            setattr(t, field, getattr(t, field) + delta)
            assert launch(t) in (tx.ERR_INVALID, tx.ERR_UNSUPPORTED), field
        # strides are re-checked at launch: another valid stride is another valid plan,
        # a short, unaligned or negative one is refused
        for field, value in (("q_sm", p.desc.head_dim - 1), ("k_sh", p.desc.k_sh + 1),
                             ("v_sz", -16), ("o_sm", p.desc.o_sm + 1)):
            t = capi.AttnPlan()
            ctypes.memmove(ctypes.byref(t), ctypes.byref(p), ctypes.sizeof(t))
            setattr(t.desc, field, value)
            assert launch(t) in (tx.ERR_INVALID, tx.ERR_UNSUPPORTED), field
    assert accepted > 150, accepted
