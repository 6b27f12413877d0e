"""ctypes mirror of include/triton_ext/{TritonExtPassInfra,tx_dot,tx_passes,tx_attn}.h."""
import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# TX_LIB_DIR: another build of the same libraries (the sanitizer build,
# triton-ext_amd/lib_asan)
LIB_DIR = os.environ.get("TX_LIB_DIR") or os.path.join(os.path.dirname(PKG_DIR), "lib")

# tx_dtype
F32, F16, BF16, I8, F8E4M3, I32, F8E5M2, F4E2M1 = 0, 1, 2, 3, 4, 5, 6, 7
DTYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", I8: "i8", F8E4M3: "f8e4m3", I32: "i32",
               F8E5M2: "f8e5m2", F4E2M1: "f4e2m1"}
# tx_scale_mode
SCALE_NONE, SCALE_ROWCOL, SCALE_BLOCK128, SCALE_MX32, SCALE_NV16 = 0, 1, 2, 3, 4
# tx_bound
BOUND_UNKNOWN, BOUND_MFMA, BOUND_HBM = 0, 1, 2
# tx_status
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_NO_DEVICE, ERR_WORKSPACE, ERR_NO_PASS = range(7)
# TX_NOALLOC_SCRATCH_BYTES: the static scratch of tx_dot_launch_noalloc, per GPU
NOALLOC_SCRATCH_BYTES = 64 << 20
# tx_kernel
(KERNEL_NONE, KERNEL_GEMM_16BIT, KERNEL_GEMM_I8, KERNEL_DECODE_I8, KERNEL_GEMM_F8,
 KERNEL_GEMM_MX, KERNEL_GEMM_MX_BF16, KERNEL_DECODE_16BIT, KERNEL_DECODE_F8) = range(9)
FLAG_NO_LOOP_SPLIT = 0x1
FLAG_B_KMAJOR = 0x2  # B stored [N][K] row-major (a transposed view in torch)
FLAG_ACCUMULATE = 0x4  # C = C + A . B (fp32 / int32 C)
# TritonPluginResult
TP_SUCCESS, TP_GENERIC_FAILURE = 0, 1
# tx_cmp_pred (arith::CmpIPredicate order)
CMP_EQ, CMP_NE, CMP_SLT, CMP_SLE, CMP_SGT, CMP_SGE, CMP_ULT, CMP_ULE, CMP_UGT, CMP_UGE = range(10)


class DotDesc(ctypes.Structure):
    _fields_ = [("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
                ("lda", ctypes.c_int64), ("ldb", ctypes.c_int64), ("ldc", ctypes.c_int64),
                ("a_type", ctypes.c_int32), ("b_type", ctypes.c_int32), ("c_type", ctypes.c_int32),
                ("scale_mode", ctypes.c_int32),
                ("block_m", ctypes.c_int32), ("block_n", ctypes.c_int32), ("block_k", ctypes.c_int32),
                ("flags", ctypes.c_int32)]


class DotPlan(ctypes.Structure):
    _fields_ = [("desc", DotDesc),
                ("flops", ctypes.c_double), ("bytes", ctypes.c_double), ("intensity", ctypes.c_double),
                ("peak_flops", ctypes.c_double), ("peak_bw", ctypes.c_double), ("ridge", ctypes.c_double),
                ("roofline_us", ctypes.c_double), ("tile_intensity", ctypes.c_double),
                ("bound", ctypes.c_int32),
                ("k_split", ctypes.c_int64), ("k_main_steps", ctypes.c_int32), ("k_tail", ctypes.c_int32),
                ("m_tiles", ctypes.c_int32), ("n_tiles", ctypes.c_int32),
                ("m_edge", ctypes.c_int32), ("n_edge", ctypes.c_int32),
                ("kernel", ctypes.c_int32), ("split_k", ctypes.c_int32),
                ("grid_x", ctypes.c_int32), ("grid_y", ctypes.c_int32), ("grid_z", ctypes.c_int32),
                ("block_threads", ctypes.c_int32), ("workspace_bytes", ctypes.c_int64),
                ("passes_run", ctypes.c_int32), ("group_m", ctypes.c_int32)]


class AttnDesc(ctypes.Structure):
    _fields_ = ([("Z", ctypes.c_int64), ("H", ctypes.c_int64), ("N_CTX", ctypes.c_int64),
                 ("head_dim", ctypes.c_int32), ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32),
                 ("sm_scale", ctypes.c_float)] +
                [(f"{t}_{s}", ctypes.c_int64) for t in "qkvo" for s in ("sz", "sh", "sm")] +
                [("block_m", ctypes.c_int32), ("block_n", ctypes.c_int32)])


class AttnPlan(ctypes.Structure):
    _fields_ = [("desc", AttnDesc), ("flops", ctypes.c_double), ("bytes", ctypes.c_double),
                ("qk_scale", ctypes.c_float), ("m_blocks", ctypes.c_int32), ("grid_x", ctypes.c_int32),
                ("block_threads", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class LoopSplit(ctypes.Structure):
    _fields_ = [("split", ctypes.c_int32), ("first_value", ctypes.c_int32),
                ("second_value", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("midp", ctypes.c_int64), ("first_trips", ctypes.c_int64),
                ("second_trips", ctypes.c_int64)]


class AIReport(ctypes.Structure):
    _fields_ = [("flops", ctypes.c_double), ("bytes", ctypes.c_double), ("intensity", ctypes.c_double),
                ("peak_flops", ctypes.c_double), ("peak_bw", ctypes.c_double), ("ridge", ctypes.c_double),
                ("roofline_us", ctypes.c_double), ("tile_intensity", ctypes.c_double),
                ("bound", ctypes.c_int32), ("block_m", ctypes.c_int32), ("block_n", ctypes.c_int32),
                ("block_k", ctypes.c_int32)]


# Every symbol the headers declare, per library (checked by the CPU tests).
EXPORTS = {
    "libTritonExtPassInfra.so": [
        "tritonAddPluginPass", "tritonRegisterPluginPass", "tritonEnumeratePluginPasses",
        "TritonExtLoadPass", "txPassManagerCreate", "txPassManagerDestroy",
        "txPassManagerAddPass", "txPassManagerSize", "txPassManagerPassName",
        "txPassManagerRun", "txRegisterPassArgument", "txPassManagerParsePipeline",
        "txReadExtConf"],
    "libloop_split.so": ["tx_loop_split_plan", "tx_loop_split_k"],
    "libarith_intensity.so": ["tx_dtype_size", "tx_dtype_bits", "tx_mi355x_peak_flops",
                              "tx_mi355x_peak_bw", "tx_arith_intensity", "tx_dot_operand_spans"],
    "libmi355x_dot.so": ["tx_dot_plan_create", "tx_dot_launch", "tx_dot_launch_noalloc",
                         "tx_get_last_error", "tx_kernel_name", "tx_device_available"],
}

_libs = {}


def lib_path(name):
    return os.path.join(LIB_DIR, name)


def load(name="libmi355x_dot.so"):
    """dlopen one of the extension libraries (RTLD_GLOBAL, like a plugin)."""
    if name in _libs:
        return _libs[name]
    path = lib_path(name)
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run __graft_entry__.build() "
                           "or `make -C triton-ext_amd`")
    L = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
    vp, i32, i64, u32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
    if name == "libTritonExtPassInfra.so":
        L.tritonAddPluginPass.argtypes = [vp, ctypes.c_char_p]
        L.tritonRegisterPluginPass.argtypes = [ctypes.c_char_p]
        L.tritonEnumeratePluginPasses.argtypes = [ctypes.POINTER(u32), ctypes.POINTER(ctypes.c_char_p)]
        L.txPassManagerCreate.restype = vp
        L.txPassManagerDestroy.argtypes = [vp]
        L.txPassManagerSize.argtypes = [vp]
        L.txPassManagerSize.restype = u32
        L.txPassManagerPassName.argtypes = [vp, u32]
        L.txPassManagerPassName.restype = ctypes.c_char_p
        L.txPassManagerRun.argtypes = [vp, ctypes.POINTER(DotPlan)]
        L.txPassManagerParsePipeline.argtypes = [vp, ctypes.c_char_p]
        L.txReadExtConf.argtypes = [ctypes.c_char_p, ctypes.c_char_p, u32, ctypes.c_char_p, u32,
                                    ctypes.c_char_p, u32]
        for f in ("tritonAddPluginPass", "tritonRegisterPluginPass", "tritonEnumeratePluginPasses",
                  "TritonExtLoadPass"):
            getattr(L, f).restype = ctypes.c_int
    elif name == "libloop_split.so":
        L.tx_loop_split_plan.argtypes = [i64, i64, i64, i32, i64, i32, i32, ctypes.POINTER(LoopSplit)]
        L.tx_loop_split_k.argtypes = [i64, i32, ctypes.POINTER(i64), ctypes.POINTER(i32),
                                      ctypes.POINTER(i32)]
    elif name == "libarith_intensity.so":
        L.tx_dtype_size.argtypes = [i32]
        L.tx_dtype_bits.argtypes = [i32]
        L.tx_mi355x_peak_flops.argtypes = [i32]
        L.tx_mi355x_peak_flops.restype = ctypes.c_double
        L.tx_mi355x_peak_bw.restype = ctypes.c_double
        L.tx_arith_intensity.argtypes = [ctypes.POINTER(DotDesc), ctypes.POINTER(AIReport)]
        L.tx_dot_operand_spans.argtypes = [ctypes.POINTER(DotDesc), ctypes.POINTER(i64),
                                           ctypes.POINTER(i64)]
    elif name == "libmi355x_dot.so":
        L.tx_dot_plan_create.argtypes = [ctypes.POINTER(DotDesc), ctypes.POINTER(DotPlan)]
        L.tx_dot_launch.argtypes = [ctypes.POINTER(DotPlan), vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
        L.tx_dot_launch_noalloc.argtypes = [ctypes.POINTER(DotPlan), vp, vp, vp, vp, vp, vp]
        L.tx_get_last_error.restype = ctypes.c_char_p
        L.tx_kernel_name.argtypes = [i32]
        L.tx_kernel_name.restype = ctypes.c_char_p
        L.tx_attn_fwd_plan.argtypes = [ctypes.POINTER(AttnDesc), ctypes.POINTER(AttnPlan)]
        L.tx_attn_fwd_launch.argtypes = [ctypes.POINTER(AttnPlan), vp, vp, vp, vp, vp, vp]
    _libs[name] = L
    return L


class TxError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"tx status {code}: {msg}")
        self.code = code


def check(rc):
    if rc != OK:
        msg = load().tx_get_last_error().decode(errors="replace")
        raise TxError(rc, msg)


def make_desc(M, N, K, a_type, c_type, b_type=None, scale_mode=SCALE_NONE, block=(0, 0, 0),
              lda=0, ldb=0, ldc=0, flags=0):
    d = DotDesc()
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = lda, ldb, ldc
    d.a_type = a_type
    d.b_type = a_type if b_type is None else b_type
    d.c_type = c_type
    d.scale_mode = scale_mode
    d.block_m, d.block_n, d.block_k = block
    d.flags = flags
    return d


def plan(desc):
    p = DotPlan()
    check(load().tx_dot_plan_create(ctypes.byref(desc), ctypes.byref(p)))
    return p


def loop_split_plan(lo, hi, step, pred, c, iv_on_rhs=False, bits=32):
    s = LoopSplit()
    rc = load("libloop_split.so").tx_loop_split_plan(lo, hi, step, pred, c, int(iv_on_rhs), bits,
                                                     ctypes.byref(s))
    if rc != OK:
        raise TxError(rc, "tx_loop_split_plan rejected its arguments")
    return s


def arith_intensity(desc):
    r = AIReport()
    rc = load("libarith_intensity.so").tx_arith_intensity(ctypes.byref(desc), ctypes.byref(r))
    if rc != OK:
        raise TxError(rc, "tx_arith_intensity rejected the descriptor")
    return r


def enumerate_passes():
    """Names from tritonEnumeratePluginPasses (two-call protocol)."""
    L = load("libTritonExtPassInfra.so")
    n = ctypes.c_uint32(0)
    if L.tritonEnumeratePluginPasses(ctypes.byref(n), None) != TP_SUCCESS:
        raise TxError(TP_GENERIC_FAILURE, "enumerate failed")
    arr = (ctypes.c_char_p * n.value)()
    if L.tritonEnumeratePluginPasses(ctypes.byref(n), arr) != TP_SUCCESS:
        raise TxError(TP_GENERIC_FAILURE, "enumerate failed")
    return [arr[i].decode() for i in range(n.value)]


def attn_plan(Z, H, N_CTX, head_dim, causal, sm_scale, dtype=F16, strides=None, block=(0, 0)):
    """Plan the fused attention forward.  strides: {"q": (sz, sh, sm), ...}
    in elements (missing tensors: packed); for dtype F8E5M2, v's are (batch,
    head, head-dim row) of its key-contiguous storage."""
    d = AttnDesc()
    d.Z, d.H, d.N_CTX, d.head_dim, d.dtype = Z, H, N_CTX, head_dim, dtype
    d.causal, d.sm_scale = int(bool(causal)), sm_scale
    for t, st in (strides or {}).items():
        for f, x in zip(("sz", "sh", "sm"), st):
            setattr(d, f"{t}_{f}", x)
    d.block_m, d.block_n = block
    p = AttnPlan()
    check(load().tx_attn_fwd_plan(ctypes.byref(d), ctypes.byref(p)))
    return p
