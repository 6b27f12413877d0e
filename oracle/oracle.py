"""ctypes wrapper of liboracle.so -- TEST INFRASTRUCTURE ONLY.

Pinned by (tests/test_oracle_cpu.py):
  * exact integer dots vs numpy int64 matmul (int8 -> int32, bit-exact);
  * fp dots vs numpy float64 matmul within fp32 rounding bounds, plus
    integer-valued fp inputs where the fp32 result is exact;
  * the Triton-interpreter golden fixtures under tests/golden/;
  * codec checks: bf16/fp16/e4m3 round trips over all bit patterns,
    known values (e4m3 max 448, min subnormal 2^-9), numpy's float16 RNE;
  * dot_scaled (tl.dot_scaled, MX): e4m3/e5m2/e8m0 decoders vs torch's
    float8 dtypes over all codes, e2m1 vs the OCP formula and the e4m3
    encoding of the same values; unit scales reduce it to the tiled fp8 dot;
    e2m1 operands equal their e4m3 re-encoding; a scale step of +1 doubles
    exactly one group's terms; golden fixtures from the interpreter running
    the dequantise-then-tl.dot form; with one bf16 operand, e4m3-valued bf16
    reduces it bit for bit to the all-MX dot, and subnormal / overflow / NaN
    scales take bf16's rounding (tests/test_mx_oracle_cpu.py);
  * fp32 -> e5m2: round to nearest even against torch's float8_e5m2 cast
    (1.6 M values), the interpreter's converter against the interpreter's
    own cast bit for bit (tests/golden/e5m2_cast_interp.npz);
  * attention (fp16, bf16, e5m2): interpreter fixtures (attn_*.npz), float64
    attention, and the LoopSplit equivalences (tests/test_attn_cpu.py).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# TX_ORACLE_LIB: another build of the same source (the sanitizer build,
# oracle/_asan/liboracle.so)
LIB_PATH = os.environ.get("TX_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

F32, F16, BF16, I8, F8E4M3, I32, F8E5M2, F4E2M1 = 0, 1, 2, 3, 4, 5, 6, 7
E8M0 = -1  # scale codec selector of mx_decode
SCALE_NONE, SCALE_ROWCOL, SCALE_BLOCK128 = 0, 1, 2
ROUND_RTZ, ROUND_RNE, ROUND_INTERP = 0, 1, 2

_lib = None


def lib():
    """Load liboracle.so (built by `make -C oracle`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle` "
                               "(or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        L.oracle_tiled_dot.restype = i32
        L.oracle_tiled_dot.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64,
                                       i32, i32, i32, i32, i32, i32, i32, i32, i64, i64, i32]
        for name in ("or_f32_to_bf16_array", "or_f32_to_e5m2_array"):
            getattr(L, name).argtypes = [vp, vp, i64, i32]
        for name in ("or_bf16_to_f32_array", "or_f32_to_f16_array", "or_f16_to_f32_array",
                     "or_f32_to_e4m3_array", "or_e4m3_to_f32_array"):
            getattr(L, name).argtypes = [vp, vp, i64]
        L.or_quantize_e4m3_groups.argtypes = [vp, i64, i64, i32, i32, vp, vp]
        L.or_mx_decode_array.argtypes = [vp, vp, i64, i32]
        L.oracle_attn_fwd.restype = i32
        L.oracle_attn_fwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i32, ctypes.c_float,
                                      i32, i32, i32, i32, i32, i32, i32]
        for name in ("oracle_dot_scaled", "oracle_dot_scaled_nv16"):
            getattr(L, name).restype = i32
            getattr(L, name).argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64,
                                         i32, i32, i32, i32, i32]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


_NP = {F32: np.float32, F16: np.uint16, BF16: np.uint16, I8: np.int8, F8E4M3: np.uint8,
       I32: np.int32}


def tiled_dot(a, b, *, a_type, c_type, block=(64, 64, 32), scale_mode=SCALE_NONE,
              sa=None, sb=None, round_mode=ROUND_RNE, tiles=None, nthreads=0, out=None,
              b_type=None):
    """Run the interpreter-equivalent tiled dot on the CPU.

    a: [M, K] array of raw element bits (uint16 for bf16/fp16, uint8 for e4m3,
    int8, float32); b: [K, N] likewise.  Returns C [M, N] (raw bits for
    16-bit outputs).  `tiles=(begin, end)` runs a subset of programs (program
    id = pid_m * tiles_n + pid_n); rows of other tiles stay as in `out`.
    round_mode: ROUND_RTZ reproduces the interpreter's truncating fp32->bf16
    cast, ROUND_RNE compiled Triton's rounding.
    """
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    M, K = a.shape
    K2, N = b.shape
    assert K == K2, (a.shape, b.shape)
    if out is None:
        out = np.zeros((M, N), dtype=_NP[c_type])
    sa_c = None if sa is None else np.ascontiguousarray(sa, dtype=np.float32)
    sb_c = None if sb is None else np.ascontiguousarray(sb, dtype=np.float32)
    t0, t1 = (0, -1) if tiles is None else tiles
    bm, bn, bk = block
    rc = lib().oracle_tiled_dot(_ptr(a), _ptr(b), _ptr(out), _ptr(sa_c), _ptr(sb_c),
                                M, N, K, K, N, N, a_type, a_type if b_type is None else b_type,
                                c_type, scale_mode,
                                round_mode, bm, bn, bk, t0, t1, nthreads)
    if rc != 0:
        raise ValueError(f"oracle_tiled_dot rejected the arguments (rc={rc})")
    return out


def f32_to_bf16(x, round_mode=ROUND_RNE):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_bf16_array(_ptr(x), _ptr(y), x.size, round_mode)
    return y


def bf16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().or_bf16_to_f32_array(_ptr(h), _ptr(y), h.size)
    return y


def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_f16_array(_ptr(x), _ptr(y), x.size)
    return y


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().or_f16_to_f32_array(_ptr(h), _ptr(y), h.size)
    return y


def f32_to_e4m3(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint8)
    lib().or_f32_to_e4m3_array(_ptr(x), _ptr(y), x.size)
    return y


def e4m3_to_f32(q):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    y = np.empty(q.shape, dtype=np.float32)
    lib().or_e4m3_to_f32_array(_ptr(q), _ptr(y), q.size)
    return y


def quantize_e4m3_groups(x, gr, gc):
    """Per-group e4m3 quantisation: scale = amax/448, q = RNE_sat(x/scale)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    q = np.empty(x.shape, dtype=np.uint8)
    s = np.empty(((rows + gr - 1) // gr, (cols + gc - 1) // gc), dtype=np.float32)
    lib().or_quantize_e4m3_groups(_ptr(x), rows, cols, gr, gc, _ptr(q), _ptr(s))
    return q, s


def mx_decode(codes, fmt):
    """Decode uint8 codes of F8E4M3 / F8E5M2 / F4E2M1 (low nibble) or E8M0
    to float64 (OCP MX semantics: e4m3 S.1111.111 and e8m0 255 are NaN)."""
    x = np.ascontiguousarray(codes, dtype=np.uint8)
    y = np.empty(x.shape, dtype=np.float64)
    lib().or_mx_decode_array(_ptr(x), _ptr(y), x.size, fmt)
    return y


def dot_scaled(a, sa, a_fmt, b, sb, b_fmt, *, K, c_type=F32, round_mode=ROUND_RNE,
               nthreads=0, nv16=False):
    """tl.dot_scaled on the CPU.

    a: uint8 [M, K] codes (e2m1: [M, K/2] packed bytes; a_fmt BF16: uint16
    bf16 bits, sa None); b: uint8 [K, N] (e2m1: [K/2, N], packed along K;
    b_fmt BF16: uint16 bits, sb None); sa: uint8 [M, K/32]; sb: uint8
    [N, K/32].  With a bf16 side the MX side is upcast to bf16 first.
    nv16: e4m3 scale codes per 16 K instead ([M, K/16], [N, K/16]).
    Returns fp32 [M, N] (c_type F32) or bf16 bits (BF16).
    """
    a = np.ascontiguousarray(a, dtype=np.uint16 if a_fmt == BF16 else np.uint8)
    b = np.ascontiguousarray(b, dtype=np.uint16 if b_fmt == BF16 else np.uint8)
    M, N = a.shape[0], b.shape[1]
    g = 16 if nv16 else 32
    sa = np.zeros((M, K // g), np.uint8) if sa is None else np.ascontiguousarray(sa, np.uint8)
    sb = np.zeros((N, K // g), np.uint8) if sb is None else np.ascontiguousarray(sb, np.uint8)
    assert sa.shape == (M, K // g) and sb.shape == (N, K // g), (sa.shape, sb.shape)
    assert a.shape[1] == (K // 2 if a_fmt == F4E2M1 else K)
    assert b.shape[0] == (K // 2 if b_fmt == F4E2M1 else K)
    out = np.zeros((M, N), dtype=np.float32 if c_type == F32 else np.uint16)
    lda = K
    fn = lib().oracle_dot_scaled_nv16 if nv16 else lib().oracle_dot_scaled
    rc = fn(_ptr(a), _ptr(b), _ptr(out), _ptr(sa), _ptr(sb), M, N, K,
            lda, N, N, a_fmt, b_fmt, c_type, round_mode, nthreads)
    if rc != 0:
        raise ValueError(f"oracle_dot_scaled rejected the arguments (rc={rc})")
    return out


def f32_to_e5m2(x, mode=ROUND_RNE):
    """fp32 -> e5m2 codes (uint8): ROUND_RNE is IEEE round to nearest even
    (overflow to inf); ROUND_INTERP the interpreter's converter."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint8)
    lib().or_f32_to_e5m2_array(_ptr(x), _ptr(y), x.size, mode)
    return y


def attn_fwd(q, k, v, *, sm_scale, causal, block=(64, 32), mode=0, dtype=F16,
             round_mode=ROUND_RNE, nthreads=0):
    """The fused-attention tutorial's forward on the CPU.

    q, k, v: uint16 fp16 (or bf16, dtype=BF16) bits, or uint8 e5m2 codes
    (dtype=F8E5M2), [Z, H, N, D] (made contiguous).  Returns (o as bits of
    the same type [Z, H, N, D], M fp32 [Z * H, N]).  block =
    (BLOCK_M, BLOCK_N); mode 0 the tutorial's split loop, 1 every block
    masked, 2 mode 0 without the blocks past the diagonal.  round_mode: bf16
    ROUND_RTZ / ROUND_RNE, e5m2 ROUND_RNE / ROUND_INTERP (fp16 is always RNE).
    """
    et = np.uint8 if dtype == F8E5M2 else np.uint16
    q = np.ascontiguousarray(q, dtype=et)
    k = np.ascontiguousarray(k, dtype=et)
    v = np.ascontiguousarray(v, dtype=et)
    Z, H, N, D = q.shape
    assert k.shape == q.shape and v.shape == q.shape
    o = np.zeros(q.shape, dtype=et)
    M = np.zeros((Z * H, N), dtype=np.float32)
    rc = lib().oracle_attn_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(M), Z, H, N, D,
                               float(sm_scale), int(causal), block[0], block[1], mode, dtype,
                               round_mode, nthreads)
    if rc != 0:
        raise ValueError(f"oracle_attn_fwd rejected the arguments (rc={rc})")
    return o, M
