"""C-ABI surface on the CPU: exports, registry, conf files, planning errors.

No kernel is launched here; launches without a gfx950 device must fail
cleanly with TX_ERR_NO_DEVICE.
"""
import ctypes
import os
import subprocess

import pytest

import triton_ext_amd as tx
from triton_ext_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
CSRC = os.path.join(ROOT, "triton-ext_amd", "csrc")
# every workspace starts with the decode kernel's 64 KiB arrival-counter region
COUNTERS = 64 << 10


def _defined_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True,
                         capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


@pytest.mark.parametrize("lib", sorted(capi.EXPORTS))
def test_library_exports(lib):
    path = capi.lib_path(lib)
    assert os.path.exists(path), f"{lib} not built"
    syms = _defined_symbols(path)
    missing = [s for s in capi.EXPORTS[lib] if s not in syms]
    assert not missing, missing
    capi.load(lib)  # and it loads


def test_header_declarations_are_exported():
    """Every function declared in include/triton_ext/*.h is exported by some library."""
    import re
    declared = set()
    for h in os.listdir(os.path.join(INC, "triton_ext")):
        text = open(os.path.join(INC, "triton_ext", h)).read()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
        text = re.sub(r"//[^\n]*", " ", text)
        declared |= set(re.findall(r"\b((?:tx|txPassManager|txRegister|txRead|triton|TritonExt)"
                                   r"[A-Za-z0-9_]*)\s*\(", text))
    declared -= {"TritonExtRegisterPassFunc", "TritonExtAddPassFunc"}
    exported = set()
    for lib in capi.EXPORTS:
        exported |= _defined_symbols(capi.lib_path(lib))
    assert declared, "no declarations found"
    assert declared <= exported, sorted(declared - exported)


def test_self_registration_and_enumeration():
    tx.load()
    names = tx.enumerate_passes()
    for n in ("loop_split", "arith_intensity", "mi355x_dot"):
        assert names.count(n) == 1, names


def test_registry_errors_and_duplicates():
    L = tx.load("libTritonExtPassInfra.so")
    assert L.tritonEnumeratePluginPasses(None, None) == capi.TP_GENERIC_FAILURE
    assert L.tritonAddPluginPass(None, b"loop_split") == capi.TP_GENERIC_FAILURE
    pm = L.txPassManagerCreate()
    assert L.tritonAddPluginPass(pm, b"no_such_extension") == capi.TP_GENERIC_FAILURE
    assert L.tritonRegisterPluginPass(b"no_such_extension") == capi.TP_GENERIC_FAILURE
    # a Python-side extension, registered twice under one name: replaced, not duplicated
    RUN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(capi.DotPlan))
    REG = ctypes.CFUNCTYPE(None)
    ADD = ctypes.CFUNCTYPE(None, ctypes.c_void_p)
    calls = []

    def run(plan):
        calls.append(plan.contents.desc.M)
        return 0
    run_c = RUN(run)
    add_c = ADD(lambda p: L.txPassManagerAddPass(ctypes.c_void_p(p), b"py-test-pass", run_c))
    reg_c = REG(lambda: calls.append("reg"))
    L.TritonExtLoadPass.argtypes = [ctypes.c_char_p, REG, ADD]
    L.txPassManagerAddPass.argtypes = [ctypes.c_void_p, ctypes.c_char_p, RUN]
    name = ctypes.create_string_buffer(b"py_test_ext")
    before = tx.enumerate_passes()
    assert L.TritonExtLoadPass(name, reg_c, add_c) == capi.TP_SUCCESS
    assert L.TritonExtLoadPass(name, reg_c, add_c) == capi.TP_SUCCESS
    after = tx.enumerate_passes()
    assert after.count("py_test_ext") == 1 and len(after) == len(before) + 1
    assert L.tritonRegisterPluginPass(b"py_test_ext") == capi.TP_SUCCESS
    assert L.tritonAddPluginPass(pm, b"py_test_ext") == capi.TP_SUCCESS
    assert L.txPassManagerSize(pm) == 1
    plan = capi.DotPlan()
    plan.desc.M = 77
    assert L.txPassManagerRun(pm, ctypes.byref(plan)) == 0
    assert calls == ["reg", 77]
    L.txPassManagerDestroy(pm)
    # keep the callbacks alive for the registry's lifetime
    test_registry_errors_and_duplicates._keep = (run_c, add_c, reg_c, name)


def test_plugin_host_harness(tmp_path):
    """A C host dlopen()s the extensions and drives them via dlsym only."""
    exe = str(tmp_path / "plugin_host")
    subprocess.run(["gcc", "-std=c11", "-O1", "-I", INC, os.path.join(ROOT, "tests", "plugin_host.c"),
                    "-o", exe, "-ldl"], check=True)
    r = subprocess.run([exe, capi.LIB_DIR], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    out = r.stdout
    assert "before_load count=0" in out
    assert "after_load count=2 loop_split arith_intensity" in out
    assert "pm size=2 tx-arith-intensity triton-loop-split" in out
    assert "plan block=256x256x64 k_split=3968 main=62 tail=32 bound=1 passes=2" in out
    assert "pipeline size=2 tx-arith-intensity triton-loop-split" in out
    assert out.strip().endswith("OK")


def test_transposes_on_host(tmp_path):
    exe = str(tmp_path / "transpose_host")
    subprocess.run(["g++", "-std=c++17", "-O2", "-I", CSRC, os.path.join(ROOT, "tests", "transpose_host.cpp"),
                    "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "OK", r.stdout + r.stderr


@pytest.mark.parametrize("fname", ["triton-ext.conf", "triton_ext.conf"])
def test_conf_reader(tmp_path, fname):
    L = tx.load("libTritonExtPassInfra.so")
    (tmp_path / fname).write_text("my_ext ; stable ; abc123\n")
    name, st, hs = (ctypes.create_string_buffer(64) for _ in range(3))
    assert L.txReadExtConf(str(tmp_path).encode(), name, 64, st, 64, hs, 64) == 0
    assert (name.value, st.value, hs.value) == (b"my_ext", b"stable", b"abc123")
    (tmp_path / fname).write_text("only_name")
    assert L.txReadExtConf(str(tmp_path).encode(), name, 64, st, 64, hs, 64) == 0
    assert (name.value, st.value, hs.value) == (b"only_name", b"experimental", b"")
    (tmp_path / fname).write_text("  \n")
    assert L.txReadExtConf(str(tmp_path).encode(), name, 64, st, 64, hs, 64) == 1
    assert L.txReadExtConf(str(tmp_path / "missing").encode(), name, 64, st, 64, hs, 64) == 1


def test_shipped_conf_files_name_the_extensions():
    L = tx.load("libTritonExtPassInfra.so")
    name = ctypes.create_string_buffer(64)
    for d, expect in (("pass/loop_split", b"loop_split"), ("pass/arith_intensity", b"arith_intensity"),
                      ("backend/mi355x", b"mi355x_dot")):
        assert L.txReadExtConf(os.path.join(CSRC, d).encode(), name, 64, None, 0, None, 0) == 0
        assert name.value == expect


def _err(desc):
    with pytest.raises(tx.TxError) as e:
        tx.plan(desc)
    return e.value.code


def test_plan_validation():
    assert _err(tx.make_desc(-1, 4, 4, tx.BF16, tx.BF16)) == tx.ERR_INVALID
    assert _err(tx.make_desc(64, 64, 64, 42, tx.BF16)) == tx.ERR_INVALID
    assert _err(tx.make_desc(64, 64, 60, tx.BF16, tx.BF16, lda=60)) == tx.ERR_INVALID  # 120 B rows
    assert _err(tx.make_desc(64, 64, 64, tx.BF16, tx.BF16, lda=32)) == tx.ERR_INVALID  # short stride
    # K and N need not fill 16-byte chunks (masked per element); row strides must
    p = tx.plan(tx.make_desc(128, 61, 68, tx.BF16, tx.BF16, lda=72, ldb=64, ldc=64))
    assert p.kernel == tx.KERNEL_GEMM_16BIT and p.k_tail == 68 % p.desc.block_k
    assert _err(tx.make_desc(128, 61, 68, tx.BF16, tx.BF16, lda=72)) == tx.ERR_INVALID  # ldb 61
    # an upcast MX B operand may have any N: its bf16 rows are N rounded up to 16 columns
    p = tx.plan(tx.make_desc(64, 72, 64, tx.BF16, tx.F32, b_type=tx.F8E4M3, ldb=80,
                             scale_mode=tx.SCALE_MX32))
    assert p.kernel == tx.KERNEL_GEMM_MX_BF16 and p.workspace_bytes == COUNTERS + 64 * 80 * 2
    assert _err(tx.make_desc(64, 64, 64, tx.BF16, tx.I32)) == tx.ERR_UNSUPPORTED
    assert _err(tx.make_desc(64, 64, 64, tx.BF16, tx.BF16, b_type=tx.F16)) == tx.ERR_UNSUPPORTED
    assert _err(tx.make_desc(64, 64, 64, tx.BF16, tx.BF16, block=(96, 64, 64))) == tx.ERR_UNSUPPORTED
    assert _err(tx.make_desc(64, 64, 64, tx.F8E4M3, tx.BF16)) == tx.ERR_UNSUPPORTED  # fp8->bf16 needs scales
    p = tx.plan(tx.make_desc(128, 64, 64, tx.BF16, tx.BF16))
    assert p.passes_run == 3 and p.kernel == tx.KERNEL_GEMM_16BIT


@pytest.mark.parametrize("M,N,K,a,c,sm,kernel", [
    (4096, 4096, 4096, tx.BF16, tx.BF16, 0, tx.KERNEL_GEMM_16BIT),
    (512, 512, 512, tx.F16, tx.F32, 0, tx.KERNEL_GEMM_16BIT),
    (1, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL, tx.KERNEL_DECODE_I8),
    (64, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL, tx.KERNEL_DECODE_I8),
    (128, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL, tx.KERNEL_DECODE_I8),
    (256, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL, tx.KERNEL_DECODE_I8),
    # past M = 256 the 8-bit tiles with split-K
    (257, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL, tx.KERNEL_GEMM_I8),
    (512, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL, tx.KERNEL_GEMM_I8),
    (513, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL, tx.KERNEL_GEMM_I8),
    # plain int8 -> int32 of decode shape: the decode kernels' int32 epilogue
    (200, 304, 256, tx.I8, tx.I32, 0, tx.KERNEL_DECODE_I8),
    (300, 304, 256, tx.I8, tx.I32, 0, tx.KERNEL_GEMM_I8),
    (2, 8192, 8192, tx.I8, tx.I32, 0, tx.KERNEL_DECODE_I8),
    (16, 8192, 8192, tx.I8, tx.I32, 0, tx.KERNEL_DECODE_I8),
    (256, 8192, 8192, tx.I8, tx.I32, 0, tx.KERNEL_DECODE_I8),
    (513, 8192, 8192, tx.I8, tx.I32, 0, tx.KERNEL_GEMM_I8),
    (4096, 4096, 4096, tx.I8, tx.I32, 0, tx.KERNEL_GEMM_I8),
    (2048, 7168, 7168, tx.F8E4M3, tx.BF16, tx.SCALE_BLOCK128, tx.KERNEL_GEMM_F8),
    # bf16 / fp16 of decode shape (M <= 96): the 16-bit decode kernel
    (1, 8192, 8192, tx.BF16, tx.BF16, 0, tx.KERNEL_DECODE_16BIT),
    (16, 8192, 8192, tx.BF16, tx.F32, 0, tx.KERNEL_DECODE_16BIT),
    (64, 4096, 4096, tx.F16, tx.F16, 0, tx.KERNEL_DECODE_16BIT),
    (33, 28672, 8192, tx.F16, tx.F32, 0, tx.KERNEL_DECODE_16BIT),
    (16, 28672, 8192, tx.BF16, tx.BF16, 0, tx.KERNEL_DECODE_16BIT),
    (16, 28672, 1024, tx.BF16, tx.BF16, 0, tx.KERNEL_DECODE_16BIT),
    (80, 8192, 8192, tx.BF16, tx.BF16, 0, tx.KERNEL_DECODE_16BIT),
    (96, 4096, 4096, tx.F16, tx.F32, 0, tx.KERNEL_DECODE_16BIT),
    (97, 8192, 8192, tx.BF16, tx.BF16, 0, tx.KERNEL_GEMM_16BIT),
    # fp8 of decode shape: the fp8 decode kernel, unscaled (fp32 C) or block-scaled
    (16, 7168, 7168, tx.F8E4M3, tx.BF16, tx.SCALE_BLOCK128, tx.KERNEL_DECODE_F8),
    (1, 8192, 8192, tx.F8E4M3, tx.F32, 0, tx.KERNEL_DECODE_F8),
    (64, 4096, 4096, tx.F8E5M2, tx.F32, 0, tx.KERNEL_DECODE_F8),
    (65, 7168, 7168, tx.F8E4M3, tx.BF16, tx.SCALE_BLOCK128, tx.KERNEL_GEMM_F8),
])
def test_kernel_choice(M, N, K, a, c, sm, kernel):
    p = tx.plan(tx.make_desc(M, N, K, a, c, scale_mode=sm))
    assert p.kernel == kernel
    assert p.grid_x > 0 and p.block_threads in (256, 512)
    if kernel == tx.KERNEL_DECODE_I8:
        # 128-column strips x row slices (one up to M = 48, of 64 rows up to 128, of 128
        # past it) x K splits cover the 256 CUs; past M = 48 the K batches are 128 rows
        bm = 256 if M > 256 else 128 if M > 128 else 64 if M > 48 else 16 * -(-M // 16)
        assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == \
            (bm, 128, 128 if M > 48 else 64)
        slices = -(-M // bm)
        assert p.grid_x == -(-N // 128) * slices * p.split_k
        if N == 8192:  # the decode shapes fill the 256 CUs
            assert p.grid_x == 256
        # a fixed 64 KiB counter region, then the int32 partials: [split][M][N] up to
        # M = 48, [split][slice][strip][block_m rows x 128 columns] past it
        rows = M if M <= 48 else slices * bm
        cols = -(-N // 4) * 4 if M <= 48 else -(-N // 128) * 128
        assert p.workspace_bytes == (65536 + p.split_k * rows * cols * 4 if p.split_k > 1 else 0)
    if kernel == tx.KERNEL_DECODE_F8:
        # the slice x 128-column strips x 128-row K batches; fp32 partials [split][strip][sr x 128]
        sr = 16 * -(-M // 16)
        assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == (sr, 128, 128)
        strips = -(-N // 128)
        assert p.grid_x == strips * p.split_k <= max(strips, 256) and p.block_threads == 256
        assert p.split_k == 1 if 2 * strips > 256 else 2 * strips * p.split_k > 256
        assert p.workspace_bytes == (65536 + p.split_k * strips * sr * 128 * 4
                                     if p.split_k > 1 else 0)
    if kernel == tx.KERNEL_DECODE_16BIT:
        # the slice of 16 ceil(M / 16) rows x strips of 64 columns (128 for slices of 32 .. 80
        # rows with N K >= 2^25) x 128-row K batches; strips x splits workgroups, at most one a
        # CU (no split once the strips alone fill them)
        sr = 16 * -(-M // 16)
        w = 128 if ((32 <= sr <= 80 and N * K >= 1 << 25)
                    or (sr == 16 and N >= 16384 and N * K >= 1 << 26)) else 64
        assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == (sr, w, 128)
        strips = -(-N // w)
        # (the largest split that keeps one workgroup a CU)
        assert p.grid_x == strips * p.split_k <= max(strips, 256) and p.block_threads == 256
        assert p.split_k == 1 if 2 * strips > 256 else 2 * strips * p.split_k > 256
        # the 64 KiB counter region, then fp32 partials: [split][strip][sr x w]
        assert p.workspace_bytes == (65536 + p.split_k * strips * sr * w * 4
                                     if p.split_k > 1 else 0)
    assert (p.split_k & (p.split_k - 1)) == 0


def test_decode_f8_plans():
    """The fp8 decode kernel: unscaled fp8 (any e4m3 / e5m2 mix) to fp32, e4m3 with 128-block
    scales to bf16 / fp32; K-major fp8 B is refused as on the tiles."""
    DF8 = tx.KERNEL_DECODE_F8
    for a, b in ((tx.F8E4M3, tx.F8E4M3), (tx.F8E4M3, tx.F8E5M2), (tx.F8E5M2, tx.F8E4M3),
                 (tx.F8E5M2, tx.F8E5M2)):
        assert tx.plan(tx.make_desc(16, 4096, 4096, a, tx.F32, b_type=b)).kernel == DF8
    for c in (tx.BF16, tx.F32):
        assert tx.plan(tx.make_desc(8, 4096, 4096, tx.F8E4M3, c,
                                    scale_mode=tx.SCALE_BLOCK128)).kernel == DF8
    assert tx.plan(tx.make_desc(16, 4096, 4096, tx.F8E4M3, tx.F32, flags=tx.FLAG_ACCUMULATE,
                                scale_mode=tx.SCALE_BLOCK128)).kernel == DF8
    # K-major B (a weight kept [N][K]): this kernel too, unscaled and block-scaled
    for c, sm in ((tx.F32, 0), (tx.BF16, tx.SCALE_BLOCK128)):
        p = tx.plan(tx.make_desc(16, 4096, 4096, tx.F8E4M3, c, scale_mode=sm,
                                 flags=tx.FLAG_B_KMAJOR))
        assert p.kernel == DF8 and (p.desc.block_m, p.desc.block_n, p.desc.block_k) == \
            (16, 128, 128)
    # an explicit 8-bit tile at decode shape runs that tile
    assert tx.plan(tx.make_desc(16, 4096, 4096, tx.F8E4M3, tx.F32,
                                block=(256, 256, 128))).kernel == tx.KERNEL_GEMM_F8
    # split-K: at least 4 batches of 128 K rows a split
    p = tx.plan(tx.make_desc(16, 7168, 7168, tx.F8E4M3, tx.BF16, scale_mode=tx.SCALE_BLOCK128))
    assert p.split_k == 4 and p.grid_x == 56 * 4  # 224 workgroups: 448 would take two rounds
    p = tx.plan(tx.make_desc(3, 1000, 300, tx.F8E4M3, tx.F32, lda=304, ldb=1008))
    assert p.split_k == 1 and p.workspace_bytes == 0 and p.grid_x == 8


def test_decode16_plans():
    """The 16-bit decode kernel: which descriptors take it, its explicit block, split-K."""
    D16 = tx.KERNEL_DECODE_16BIT
    # K-major B (q @ k.T at decode, or a weight kept [N][K]) too, ldb defaulting to K
    p = tx.plan(tx.make_desc(16, 4096, 4000, tx.BF16, tx.BF16, lda=4000,
                             flags=tx.FLAG_B_KMAJOR))
    assert p.kernel == D16 and p.desc.ldb == 4000 and (p.desc.block_m, p.desc.block_k) == (16, 128)
    assert tx.plan(tx.make_desc(64, 300, 72, tx.F16, tx.F32, ldb=80,
                                flags=tx.FLAG_B_KMAJOR | tx.FLAG_ACCUMULATE)).kernel == D16
    # mixed operand types: not this kernel
    assert _err(tx.make_desc(16, 4096, 4096, tx.BF16, tx.F16)) == tx.ERR_UNSUPPORTED
    # an explicit GEMM tile at decode shape runs that tile; the decode block at M > 96 is refused
    assert tx.plan(tx.make_desc(16, 4096, 4096, tx.BF16, tx.BF16,
                                block=(64, 64, 32))).kernel == tx.KERNEL_GEMM_16BIT
    assert tx.plan(tx.make_desc(16, 4096, 4096, tx.BF16, tx.BF16,
                                block=(16, 64, 128))).kernel == D16
    assert tx.plan(tx.make_desc(80, 4096, 4096, tx.BF16, tx.BF16,
                                block=(80, 64, 128))).kernel == D16
    assert _err(tx.make_desc(112, 4096, 4096, tx.BF16, tx.BF16,
                             block=(112, 64, 128))) == tx.ERR_UNSUPPORTED
    # tl.dot(a, b, acc) with an fp32 acc
    p = tx.plan(tx.make_desc(8, 1000, 3000, tx.BF16, tx.F32, flags=tx.FLAG_ACCUMULATE))
    assert p.kernel == D16 and p.split_k == 4 and p.grid_x == 16 * 4
    # K = 0 and a K that fills no whole batch: one split
    for K in (0, 100):
        p = tx.plan(tx.make_desc(4, 4096, K, tx.F16, tx.F16, lda=-(-K // 8) * 8))
        assert p.kernel == D16 and p.split_k == 1 and p.workspace_bytes == 0
    # split-K: every split owns at least 4 batches of 128 K rows
    p = tx.plan(tx.make_desc(16, 1024, 8192, tx.BF16, tx.BF16))
    assert p.split_k == 16 and p.grid_x == 256
    p = tx.plan(tx.make_desc(16, 1024, 2048, tx.BF16, tx.BF16))
    assert p.split_k == 4


def test_b_kmajor_plans():
    """K-major B (q @ k.T): bf16/fp16 on the 256x256x64 tile, int8 -> int32 and unscaled
    fp8 on the 256x256x128 tile, and at decode shapes on the decode kernels; ldb defaulting
    to K."""
    p = tx.plan(tx.make_desc(512, 384, 192, tx.BF16, tx.F32, flags=tx.FLAG_B_KMAJOR))
    assert p.kernel == tx.KERNEL_GEMM_16BIT
    assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == (256, 256, 64)
    assert p.desc.ldb == 192 and p.block_threads == 256
    assert _err(tx.make_desc(64, 64, 64, tx.BF16, tx.BF16, ldb=32,
                             flags=tx.FLAG_B_KMAJOR)) == tx.ERR_INVALID  # ldb < K
    assert _err(tx.make_desc(64, 64, 64, tx.BF16, tx.BF16, block=(128, 128, 64),
                             flags=tx.FLAG_B_KMAJOR)) == tx.ERR_UNSUPPORTED
    for a, b, c, kern in ((tx.I8, tx.I8, tx.I32, tx.KERNEL_GEMM_I8),
                          (tx.F8E4M3, tx.F8E4M3, tx.F32, tx.KERNEL_GEMM_F8),
                          (tx.F8E5M2, tx.F8E4M3, tx.F32, tx.KERNEL_GEMM_F8),
                          (tx.F8E4M3, tx.F8E5M2, tx.F32, tx.KERNEL_GEMM_F8),
                          (tx.F8E5M2, tx.F8E5M2, tx.F32, tx.KERNEL_GEMM_F8)):
        p = tx.plan(tx.make_desc(600, 300, 200, a, c, b_type=b, lda=208, ldb=208,
                                 flags=tx.FLAG_B_KMAJOR))
        assert p.kernel == kern and p.desc.ldb == 208
        assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == (256, 256, 128)
        # M <= 64: the 8-bit decode kernel, or the 256 tile by name
        p = tx.plan(tx.make_desc(16, 300, 200, a, c, b_type=b, lda=208, ldb=208,
                                 flags=tx.FLAG_B_KMAJOR))
        assert p.kernel == tx.KERNEL_DECODE_F8 and p.desc.ldb == 208
        assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == (16, 128, 128)
        assert tx.plan(tx.make_desc(16, 300, 200, a, c, b_type=b, lda=208, ldb=208,
                                    block=(256, 256, 128), flags=tx.FLAG_B_KMAJOR)).kernel == kern
    # W8A8 and block-scaled fp8 (weights kept [N][K]): the 8-bit decode kernel at M <= 64;
    # int8 (W8A8, int32) on the row kernel to M = 256; the 256 tile beyond
    for a, c, sm, kern in ((tx.I8, tx.BF16, tx.SCALE_ROWCOL, tx.KERNEL_GEMM_I8),
                           (tx.I8, tx.I32, 0, tx.KERNEL_GEMM_I8),
                           (tx.F8E4M3, tx.BF16, tx.SCALE_BLOCK128, tx.KERNEL_GEMM_F8),
                           (tx.F8E4M3, tx.F32, tx.SCALE_BLOCK128, tx.KERNEL_GEMM_F8)):
        i8 = a == tx.I8
        for M, want, blk in ((16, tx.KERNEL_DECODE_F8, (16, 128, 128)),
                             (100, tx.KERNEL_DECODE_I8 if i8 else kern,
                              (64, 128, 128) if i8 else (256, 256, 128)),
                             (200, tx.KERNEL_DECODE_I8 if i8 else kern,
                              (128, 128, 128) if i8 else (256, 256, 128)),
                             (300, kern, (256, 256, 128)), (600, kern, (256, 256, 128))):
            p = tx.plan(tx.make_desc(M, 512, 512, a, c, scale_mode=sm, flags=tx.FLAG_B_KMAJOR))
            assert p.kernel == want and (p.desc.block_m, p.desc.block_n, p.desc.block_k) == blk
    # the K-interleaved int8 decode kernel (decode_i8.h) has no K-major form
    assert _err(tx.make_desc(100, 512, 512, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL,
                             block=(64, 128, 64), flags=tx.FLAG_B_KMAJOR)) == tx.ERR_UNSUPPORTED
    # the other 8-bit tiles (256 x 224; register-staged 128 x 128, which 128 x 128 x 128
    # names past M = 256) have no K-major form
    for M, a, c, sm, blk in ((300, tx.I8, tx.BF16, tx.SCALE_ROWCOL, (128, 128, 128)),
                             (16, tx.F8E4M3, tx.BF16, tx.SCALE_BLOCK128, (256, 224, 128)),
                             (300, tx.I8, tx.I32, 0, (128, 128, 128)),
                             (16, tx.I8, tx.I32, 0, (256, 224, 128))):
        assert _err(tx.make_desc(M, 256, 256, a, c, scale_mode=sm, block=blk,
                                 flags=tx.FLAG_B_KMAJOR)) == tx.ERR_UNSUPPORTED
    assert _err(tx.make_desc(64, 64, 64, tx.BF16, tx.BF16, flags=0x10)) == tx.ERR_INVALID


def test_mx_plans():
    """tl.dot_scaled (TX_SCALE_MX32): fp8 / fp4 on the 256x256 tile, 128 bytes of K per step."""
    MX = tx.SCALE_MX32
    for a, b, c in ((tx.F8E4M3, tx.F8E4M3, tx.F32), (tx.F8E4M3, tx.F8E5M2, tx.BF16),
                    (tx.F8E5M2, tx.F8E4M3, tx.F32), (tx.F8E5M2, tx.F8E5M2, tx.BF16)):
        p = tx.plan(tx.make_desc(1000, 528, 4000, a, c, b_type=b, scale_mode=MX))
        assert p.kernel == tx.KERNEL_GEMM_MX and p.block_threads == 512
        assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == (256, 256, 128)
        assert p.k_main_steps == 4000 // 128 and p.k_tail == 4000 % 128
        assert p.grid_x == 4 * 3
        # algorithmic bytes: fp8 operands, one e8m0 byte per 32 K of each row
        # and column, C once
        assert p.bytes == 1000 * 4000 + 4000 * 528 + (1000 + 528) * 125 + \
            1000 * 528 * (4 if c == tx.F32 else 2)
        assert p.peak_flops == pytest.approx(5033.2e12)
    p = tx.plan(tx.make_desc(512, 256, 1024, tx.F4E2M1, tx.F32, scale_mode=MX))
    assert p.kernel == tx.KERNEL_GEMM_MX
    assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == (256, 256, 256)
    assert p.desc.lda == 1024 and p.desc.ldb == 256
    assert p.bytes == 512 * 512 + 512 * 256 + (512 + 256) * 32 + 512 * 256 * 4
    assert p.peak_flops == pytest.approx(10066.4e12)
    assert tx.load("libarith_intensity.so").tx_dtype_bits(tx.F4E2M1) == 4
    assert tx.load("libarith_intensity.so").tx_dtype_size(tx.F4E2M1) == 0

    def err(**kw):
        d = dict(M=64, N=64, K=256, a_type=tx.F8E4M3, c_type=tx.F32, scale_mode=MX)
        d.update(kw)
        return _err(tx.make_desc(d.pop("M"), d.pop("N"), d.pop("K"), d.pop("a_type"),
                                 d.pop("c_type"), **d))
    assert err(K=272) == tx.ERR_UNSUPPORTED          # K % 32
    assert err(b_type=tx.F4E2M1, K=256) == tx.ERR_UNSUPPORTED  # fp8 with fp4
    assert err(c_type=tx.F16) == tx.ERR_UNSUPPORTED
    assert err(a_type=tx.I8, c_type=tx.BF16) == tx.ERR_UNSUPPORTED
    assert err(flags=tx.FLAG_B_KMAJOR) == tx.ERR_UNSUPPORTED
    assert err(a_type=tx.F4E2M1, scale_mode=tx.SCALE_NONE) == tx.ERR_UNSUPPORTED
    assert err(scale_mode=5) == tx.ERR_INVALID
    assert err(scale_mode=tx.SCALE_NV16) == tx.ERR_UNSUPPORTED  # e4m3 values, e4m3 scales
    assert err(a_type=tx.F4E2M1, K=256, lda=264) == tx.ERR_INVALID  # 132-byte rows
    # the fp32 block-scaled mode keeps rejecting e5m2 (e4m3 only)
    assert err(a_type=tx.F8E5M2, scale_mode=tx.SCALE_BLOCK128) == tx.ERR_UNSUPPORTED
    # MX x bf16: the MX operand upcast into the workspace, then the bf16 tile
    for a, b in ((tx.BF16, tx.F4E2M1), (tx.BF16, tx.F8E4M3), (tx.F8E5M2, tx.BF16),
                 (tx.F4E2M1, tx.BF16)):
        p = tx.plan(tx.make_desc(1000, 528, 4000, a, tx.F32, b_type=b, scale_mode=MX))
        assert p.kernel == tx.KERNEL_GEMM_MX_BF16
        q = tx.plan(tx.make_desc(1000, 528, 4000, tx.BF16, tx.F32))  # the bf16 dot's tile
        assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == \
            (q.desc.block_m, q.desc.block_n, q.desc.block_k)
        assert (p.k_main_steps, p.k_tail, p.grid_x) == (q.k_main_steps, q.k_tail, q.grid_x)
        assert (p.split_k, p.grid_y) == (q.split_k, q.grid_y) and q.split_k > 1
        mx_elems = 4000 * 528 if b != tx.BF16 else 1000 * 4000
        # the upcast operand, then (after it) the bf16 dot's split-K partials
        assert p.workspace_bytes == COUNTERS + (mx_elems * 2 + 255) // 256 * 256 + \
            q.workspace_bytes - COUNTERS
        bits = {tx.BF16: 16, tx.F4E2M1: 4, tx.F8E4M3: 8, tx.F8E5M2: 8}
        scale_rows = 528 if b != tx.BF16 else 1000  # only the MX side is scaled
        assert p.bytes == 1000 * 4000 * bits[a] / 8 + 4000 * 528 * bits[b] / 8 + \
            scale_rows * 125 + 1000 * 528 * 4
        assert p.peak_flops == pytest.approx(2516.6e12)
    assert err(a_type=tx.BF16, b_type=tx.BF16) == tx.ERR_UNSUPPORTED  # bf16 on both sides
    assert err(a_type=tx.F16, b_type=tx.F4E2M1) == tx.ERR_UNSUPPORTED  # fp16 side


def test_nv16_plans():
    """e4m3 scales per 16 (TX_SCALE_NV16): e2m1 sides upcast to bf16, the bf16 tile."""
    NV = tx.SCALE_NV16
    p = tx.plan(tx.make_desc(512, 256, 1024, tx.F4E2M1, tx.F32, b_type=tx.F4E2M1, scale_mode=NV))
    assert p.kernel == tx.KERNEL_GEMM_MX_BF16
    q = tx.plan(tx.make_desc(512, 256, 1024, tx.BF16, tx.F32))  # the bf16 dot it runs
    assert (p.split_k, p.grid_x, p.grid_y) == (q.split_k, q.grid_x, q.grid_y)
    partials = q.workspace_bytes - COUNTERS if q.split_k > 1 else 0
    assert p.workspace_bytes == COUNTERS + 512 * 1024 * 2 + 1024 * 256 * 2 + partials  # as bf16
    assert p.bytes == 512 * 512 + 512 * 256 + (512 + 256) * 64 + 512 * 256 * 4
    assert p.peak_flops == pytest.approx(2516.6e12)
    p = tx.plan(tx.make_desc(512, 256, 1024, tx.BF16, tx.F32, b_type=tx.F4E2M1, scale_mode=NV))
    assert p.workspace_bytes == COUNTERS + 1024 * 256 * 2 + partials
    assert _err(tx.make_desc(64, 64, 256, tx.F8E4M3, tx.F32, scale_mode=NV)) == tx.ERR_UNSUPPORTED
    assert _err(tx.make_desc(64, 64, 256, tx.F4E2M1, tx.F32, scale_mode=5)) == tx.ERR_INVALID


def test_accumulate_plans():
    """TX_FLAG_ACCUMULATE: fp32 / int32 C only; C counts twice in the bytes."""
    p = tx.plan(tx.make_desc(1024, 1024, 1024, tx.BF16, tx.F32, flags=tx.FLAG_ACCUMULATE))
    q = tx.plan(tx.make_desc(1024, 1024, 1024, tx.BF16, tx.F32))
    assert p.bytes == q.bytes + 1024 * 1024 * 4 and p.kernel == q.kernel
    # int32 C accumulates on the decode kernels too (M <= 512) and on the 8-bit tiles
    assert tx.plan(tx.make_desc(64, 128, 256, tx.I8, tx.I32,
                                flags=tx.FLAG_ACCUMULATE)).kernel == tx.KERNEL_DECODE_I8
    assert tx.plan(tx.make_desc(1024, 128, 256, tx.I8, tx.I32,
                                flags=tx.FLAG_ACCUMULATE)).kernel == tx.KERNEL_GEMM_I8
    assert _err(tx.make_desc(256, 256, 256, tx.BF16, tx.BF16,
                             flags=tx.FLAG_ACCUMULATE)) == tx.ERR_UNSUPPORTED
    assert _err(tx.make_desc(16, 8192, 8192, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL,
                             flags=tx.FLAG_ACCUMULATE)) == tx.ERR_UNSUPPORTED  # W8A8: bf16 C
    assert _err(tx.make_desc(64, 64, 64, tx.BF16, tx.F32, flags=0x8)) == tx.ERR_INVALID


def test_fp8_e5m2_plans():
    """tt.dot over fp8 pairs with e5m2 (any mix, fp32 C): the 256x256 8-bit tile."""
    for a, b in ((tx.F8E5M2, tx.F8E5M2), (tx.F8E4M3, tx.F8E5M2), (tx.F8E5M2, tx.F8E4M3)):
        p = tx.plan(tx.make_desc(300, 272, 400, a, tx.F32, b_type=b))
        assert p.kernel == tx.KERNEL_GEMM_F8
        assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == (256, 256, 128)
        assert p.peak_flops == pytest.approx(5033.2e12)
        assert _err(tx.make_desc(300, 272, 400, a, tx.BF16, b_type=b)) == tx.ERR_UNSUPPORTED
        assert _err(tx.make_desc(256, 256, 256, a, tx.F32, b_type=b,
                                 block=(128, 128, 128))) == tx.ERR_UNSUPPORTED
    assert _err(tx.make_desc(64, 64, 128, tx.F8E5M2, tx.F32, b_type=tx.BF16)) == tx.ERR_UNSUPPORTED


def test_dot_scaled_argument_checks():
    """Host mirror of tl.dot_scaled: Triton's shape checks (no device needed)."""
    import torch
    a = torch.zeros(64, 128, dtype=torch.uint8)
    b = torch.zeros(128, 32, dtype=torch.uint8)
    sa = torch.zeros(64, 4, dtype=torch.uint8)
    sb = torch.zeros(32, 4, dtype=torch.uint8)
    with pytest.raises(ValueError, match="NYI: lhs_format"):
        tx.dot_scaled(a, sa, "e3m4", b, sb, "e4m3")
    with pytest.raises(NotImplementedError):
        tx.dot_scaled(a, sa, "fp16", b, sb, "e4m3")
    with pytest.raises(ValueError, match=r"rhs_scale must be a tensor of shape \[32, 4\]"):
        tx.dot_scaled(a, sa, "e4m3", b, sb.t().contiguous(), "e4m3")
    with pytest.raises(ValueError, match="Reduction dimension"):
        tx.dot_scaled(a, sa, "e2m1", b, sb, "e4m3")  # lhs packs 256, rhs 128
    with pytest.raises(ValueError, match="acc must be fp32"):
        tx.dot_scaled(a, sa, "e4m3", b, sb, "e4m3", acc=torch.zeros(64, 32, dtype=torch.int32))
    # a scale of None is accepted (unit scales); shapes are still checked
    with pytest.raises(ValueError, match="Reduction dimension"):
        tx.dot_scaled(a, None, "e2m1", b, None, "e4m3")
    # bf16 operands: a torch.bfloat16 tensor and no scale; fp16 is not built
    abf = torch.zeros(64, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no scale"):
        tx.dot_scaled(abf, sa, "bf16", b, sb, "e4m3")
    with pytest.raises(ValueError, match="no scale"):
        tx.dot_scaled(a, None, "bf16", b, sb, "e4m3")  # uint8 tensor named bf16
    with pytest.raises(NotImplementedError):
        tx.dot_scaled(abf.half(), None, "fp16", b, sb, "e4m3")
    with pytest.raises(NotImplementedError):
        tx.dot_scaled(abf, None, "bf16", abf.t().contiguous(), None, "bf16")


def test_launch_without_device_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("device present")
    L = tx.load()
    p = tx.plan(tx.make_desc(64, 64, 64, tx.BF16, tx.BF16))
    buf = ctypes.create_string_buffer(64 * 64 * 2 + 16)
    addr = (ctypes.addressof(buf) + 15) & ~15
    rc = L.tx_dot_launch(ctypes.byref(p), addr, addr, addr, None, None, None, 0, None)
    assert rc == tx.ERR_NO_DEVICE
    assert b"gfx950" in L.tx_get_last_error()
    assert L.tx_device_available() == 0
    # argument errors are reported before the device is touched
    assert L.tx_dot_launch(None, addr, addr, addr, None, None, None, 0, None) == tx.ERR_INVALID
    assert L.tx_dot_launch(ctypes.byref(p), None, addr, addr, None, None, None, 0, None) == tx.ERR_INVALID
    assert L.tx_dot_launch(ctypes.byref(p), addr + 2, addr, addr, None, None, None, 0, None) == tx.ERR_INVALID


def test_operand_spans_and_32bit_tiles():
    """The 256-wide tiles address A and B through 32-bit buffer offsets.  An
    operand spanning 2^31 bytes or more gets a 128x128 tile (64-bit
    addresses) from the tile choice, and an explicit 256-wide tile is
    rejected at plan time, before any launch."""
    spans = tx.load("libarith_intensity.so").tx_dot_operand_spans
    a, b = ctypes.c_int64(), ctypes.c_int64()

    def span(desc):
        assert spans(ctypes.byref(desc), ctypes.byref(a), ctypes.byref(b)) == tx.OK
        return a.value, b.value
    assert span(tx.make_desc(300, 200, 100, tx.BF16, tx.F32, lda=104, ldb=208)) == \
        ((299 * 104 + 100) * 2, (99 * 208 + 200) * 2)
    assert span(tx.make_desc(64, 32, 128, tx.BF16, tx.F32, flags=tx.FLAG_B_KMAJOR)) == \
        (64 * 128 * 2, 32 * 128 * 2)
    assert span(tx.make_desc(8, 16, 64, tx.F4E2M1, tx.F32, scale_mode=tx.SCALE_MX32)) == \
        (8 * 64 // 2, 32 * 16)
    assert span(tx.make_desc(0, 16, 64, tx.I8, tx.I32))[0] == 0
    # bf16 32768 x 32768: 2 GiB each, exactly the first span the tiles cannot take
    big = tx.make_desc(32768, 32768, 32768, tx.BF16, tx.BF16)
    assert span(big) == (1 << 31, 1 << 31)
    p = tx.plan(big)
    assert (p.desc.block_m, p.desc.block_n) == (128, 128) and p.kernel == tx.KERNEL_GEMM_16BIT
    assert _err(tx.make_desc(32768, 32768, 32768, tx.BF16, tx.BF16,
                             block=(256, 256, 64))) == tx.ERR_UNSUPPORTED
    assert b"32-bit" in tx.load().tx_get_last_error()
    # just under 2 GiB each: the 256-wide tile
    d = tx.make_desc(32767, 32760, 32768, tx.BF16, tx.BF16, ldb=32768)
    assert span(d) == (32767 * 32768 * 2, (1 << 31) - 16)
    p = tx.plan(d)
    assert p.desc.block_m == 256
    # int8 4 GiB A (the advisor's case): 128x128 register tile; explicit 256 rejected
    p = tx.plan(tx.make_desc(131072, 4096, 32768, tx.I8, tx.I32))
    assert (p.desc.block_m, p.desc.block_n) == (128, 128) and p.kernel == tx.KERNEL_GEMM_I8
    assert _err(tx.make_desc(131072, 4096, 32768, tx.I8, tx.I32,
                             block=(256, 256, 128))) == tx.ERR_UNSUPPORTED
    # fp8 4 GiB A, block-scaled: the 128x128 fp8 tile
    p = tx.plan(tx.make_desc(65536, 4096, 65536, tx.F8E4M3, tx.BF16,
                             scale_mode=tx.SCALE_BLOCK128))
    assert (p.desc.block_m, p.desc.block_n) == (128, 128)
    # K-major B and MX have only 256-wide tiles: rejected
    assert _err(tx.make_desc(65536, 4096, 32768, tx.BF16, tx.F32,
                             flags=tx.FLAG_B_KMAJOR)) == tx.ERR_UNSUPPORTED
    assert _err(tx.make_desc(65536, 256, 65536, tx.F8E4M3, tx.F32,
                             scale_mode=tx.SCALE_MX32)) == tx.ERR_UNSUPPORTED
    # the W8A8 decode kernel uses 64-bit addresses: B of 4 GiB plans
    p = tx.plan(tx.make_desc(16, 65536, 65536, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL))
    assert p.kernel == tx.KERNEL_DECODE_I8


def test_nv16_needs_whole_scale_groups():
    """e4m3 scales per 16: K % 16 == 0, also when the other side is bf16."""
    NV = tx.SCALE_NV16
    for K in (24, 40, 1032):
        assert _err(tx.make_desc(64, 64, K, tx.BF16, tx.F32, b_type=tx.F4E2M1,
                                 scale_mode=NV)) == tx.ERR_UNSUPPORTED
        assert b"K % 16" in tx.load().tx_get_last_error()
    assert tx.plan(tx.make_desc(64, 64, 32, tx.BF16, tx.F32, b_type=tx.F4E2M1,
                                scale_mode=NV)).kernel == tx.KERNEL_GEMM_MX_BF16


def test_plan_and_acc_must_agree():
    """dot() / dot_scaled() with a caller's plan: FLAG_ACCUMULATE set exactly
    when acc is given (checked before anything reaches the device)."""
    import torch
    a = torch.zeros(64, 64, dtype=torch.bfloat16)
    acc = torch.zeros(64, 64, dtype=torch.float32)
    plain = tx.plan(tx.make_desc(64, 64, 64, tx.BF16, tx.F32))
    accum = tx.plan(tx.make_desc(64, 64, 64, tx.BF16, tx.F32, flags=tx.FLAG_ACCUMULATE))
    with pytest.raises(ValueError, match="disagree on acc"):
        tx.dot(a, a, acc=acc, plan=plain)
    with pytest.raises(ValueError, match="disagree on acc"):
        tx.dot(a, a, out_dtype=torch.float32, plan=accum)
    q = torch.zeros(64, 64, dtype=torch.uint8)
    s = torch.full((64, 2), 127, dtype=torch.uint8)
    mxp = tx.plan(tx.make_desc(64, 64, 64, tx.F8E4M3, tx.F32, scale_mode=tx.SCALE_MX32))
    with pytest.raises(ValueError, match="disagree on acc"):
        tx.dot_scaled(q, s, "e4m3", q, s, "e4m3", acc=acc, plan=mxp)


def test_noalloc_rejects_oversized_workspace():
    """tx_dot_launch_noalloc takes no workspace: a plan needing more than the static scratch
    holds fails with TX_ERR_WORKSPACE before the device is touched."""
    L = tx.load()
    buf = ctypes.create_string_buffer(4096 + 16)
    addr = (ctypes.addressof(buf) + 15) & ~15
    # MX x bf16 at 8192^2: the upcast B is 128 MiB
    p = tx.plan(tx.make_desc(256, 8192, 8192, tx.BF16, tx.F32, b_type=tx.F8E4M3,
                             scale_mode=tx.SCALE_MX32))
    assert p.workspace_bytes > capi.NOALLOC_SCRATCH_BYTES
    rc = L.tx_dot_launch_noalloc(ctypes.byref(p), addr, addr, addr, None, addr, None)
    assert rc == tx.ERR_WORKSPACE and b"no-allocation scratch" in L.tx_get_last_error()
    # decode partials beyond the scratch: M = 64, N = 131072 (4 splits x 32 MiB)
    p = tx.plan(tx.make_desc(64, 131072, 8192, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL))
    if p.workspace_bytes > capi.NOALLOC_SCRATCH_BYTES:
        rc = L.tx_dot_launch_noalloc(ctypes.byref(p), addr, addr, addr, addr, addr, None)
        assert rc == tx.ERR_WORKSPACE
    # within the scratch: argument checks pass, then no device
    import torch
    if not torch.cuda.is_available():
        p = tx.plan(tx.make_desc(16, 8192, 8192, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL))
        rc = L.tx_dot_launch_noalloc(ctypes.byref(p), addr, addr, addr, addr, addr, None)
        assert rc == tx.ERR_NO_DEVICE
