"""ctypes binding of libc3hip.so (include/c3hip.h).

Every structure below mirrors its C counterpart field for field; `check_abi()`
compares the sizes against the library's own `c3h_abi_sizes()` so a layout
drift fails loudly at import time instead of corrupting kernel arguments.

The library is the only compute path.  If it is missing, `lib()` raises: no
operation in this package falls back to NumPy or any other CPU code.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Optional

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libc3hip.so"

MAX_RANK = 8
EW_MAX_IN = 8
EW_MAX_INST = 16

# dtype codes (enum c3h_dtype)
F32, F16, BF16, I8, I32, I64, U8, BOOL, F64 = range(9)

# elementwise opcodes (enum c3h_ew_opcode)
EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_RELU, EW_ERF, EW_ERF_AS, EW_SQRT, EW_EXP, EW_RECIP, \
    EW_MAX, EW_MIN, EW_NEG, EW_ADD_IMM, EW_MUL_IMM, EW_COPY = range(16)

# timeline op kinds (enum c3h_op_kind)
OP_NOP, OP_EVENT_RECORD, OP_EVENT_WAIT, OP_COPY = 0, 1, 2, 3
OP_FILL, OP_CAST, OP_EW, OP_STRIDED_COPY, OP_REDUCE, OP_SOFTMAX, OP_LAYERNORM, OP_BATCHNORM, \
    OP_GATHER, OP_ARGMAX, OP_IM2COL, OP_LAYOUT, OP_MAXPOOL, OP_GEMM, OP_CONV, OP_ATTN_SCORES, \
    OP_FLASH, OP_QUANTIZE, OP_QGEMM, OP_DEQUANTIZE, OP_BNFOLD, OP_PACK, OP_CONV_POOL, OP_QUANT_FP8, \
    OP_GEMM_FP8, OP_SPLITK, OP_QUANT_MXFP4, OP_GEMM_W4A16, OP_ARGMAX_FINISH, OP_NONFINITE = range(10, 40)

vp = C.c_void_p
i32 = C.c_int32
i64 = C.c_int64
f32 = C.c_float


class Props(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("arch", C.c_char * 64), ("compute_units", i32),
                ("warp_size", i32), ("max_threads_per_block", i32), ("max_block_dim_x", i32),
                ("max_grid_dim_x", i32), ("lds_bytes_per_block", i32), ("clock_khz", i32),
                ("memory_clock_khz", i32), ("memory_bus_width", i32), ("l2_bytes", i32),
                ("total_memory_bytes", i64), ("major", i32), ("minor", i32)]


class FillArgs(C.Structure):
    _fields_ = [("out", vp), ("count", i64), ("dtype", i32), ("pad_", i32), ("value", C.c_double)]


class CastArgs(C.Structure):
    _fields_ = [("in_", vp), ("out", vp), ("count", i64), ("in_dtype", i32), ("out_dtype", i32)]


class EwInst(C.Structure):
    _fields_ = [("op", i32), ("a", i32), ("b", i32), ("pad_", i32), ("imm", f32), ("pad2_", f32)]


class EwArgs(C.Structure):
    _fields_ = [("in_", vp * EW_MAX_IN), ("in_dtype", i32 * EW_MAX_IN),
                ("stride", (i64 * MAX_RANK) * EW_MAX_IN), ("out", vp), ("out_dtype", i32),
                ("rank", i32), ("shape", i64 * MAX_RANK), ("n_in", i32), ("n_inst", i32),
                ("inst", EwInst * EW_MAX_INST)]


class CopyArgs(C.Structure):
    _fields_ = [("in_", vp), ("out", vp), ("elem_bytes", i32), ("rank", i32),
                ("shape", i64 * MAX_RANK), ("in_stride", i64 * MAX_RANK), ("in_offset", i64)]


class ReduceArgs(C.Structure):
    _fields_ = [("in_", vp), ("out", vp), ("outer", i64), ("reduce", i64), ("inner", i64),
                ("kind", i32), ("in_dtype", i32), ("out_dtype", i32), ("pad_", i32)]


class SoftmaxArgs(C.Structure):
    _fields_ = [("in_", vp), ("out", vp), ("outer", i64), ("axis", i64), ("inner", i64),
                ("in_dtype", i32), ("out_dtype", i32)]


class LayerNormArgs(C.Structure):
    _fields_ = [("x", vp), ("residual", vp), ("scale", vp), ("bias", vp), ("out", vp),
                ("mean_out", vp), ("invstd_out", vp), ("rows", i64), ("cols", i64),
                ("epsilon", f32), ("x_dtype", i32), ("out_dtype", i32), ("out_scale", f32), ("out_zero", i32),
                ("pad_", i32)]


class BatchNormArgs(C.Structure):
    _fields_ = [("x", vp), ("scale", vp), ("bias", vp), ("mean", vp), ("var", vp), ("out", vp),
                ("n", i64), ("c", i64), ("hw", i64), ("epsilon", f32), ("pad_", i32)]


class BnFoldArgs(C.Structure):
    _fields_ = [("w", vp), ("conv_bias", vp), ("scale", vp), ("bias", vp), ("mean", vp),
                ("var", vp), ("w_out", vp), ("b_out", vp), ("out_channels", i64),
                ("per_channel", i64), ("epsilon", f32), ("pad_", i32)]


class GatherArgs(C.Structure):
    _fields_ = [("data", vp), ("indices", vp), ("out", vp), ("error_flag", vp), ("outer", i64),
                ("axis_dim", i64), ("inner", i64), ("n_indices", i64), ("elem_bytes", i32),
                ("dtype", i32), ("addend", vp), ("addend_rows", i64), ("addend_dtype", i32),
                ("pad_", i32)]


class ArgmaxArgs(C.Structure):
    _fields_ = [("in_", vp), ("out", vp), ("rows", i64), ("cols", i64), ("in_dtype", i32),
                ("pad_", i32)]


class NonfiniteArgs(C.Structure):
    _fields_ = [("x", vp), ("flag", vp), ("count", i64), ("dtype", i32), ("pad_", i32)]


class ArgmaxFinishArgs(C.Structure):
    _fields_ = [("parts", vp), ("in_", vp), ("out", vp), ("rows", i64), ("cols", i64), ("n_parts", i64),
                ("ld", i64), ("in_ld", i64), ("in_dtype", i32), ("pad_", i32)]


class Im2colArgs(C.Structure):
    _fields_ = [(n, i32) for n in ("n", "c", "h", "w", "kh", "kw", "sh", "sw", "pad_top",
                                   "pad_left", "dh", "dw", "ho", "wo", "dtype", "pad_")]
    _fields_ = [("x", vp), ("out", vp)] + _fields_


class LayoutArgs(C.Structure):
    _fields_ = [("in_", vp), ("out", vp)] + [(n, i32) for n in (
        "n", "c", "h", "w", "c_pad", "direction", "in_dtype", "out_dtype")]


class PoolArgs(C.Structure):
    _fields_ = [("x", vp), ("out", vp)] + [(n, i32) for n in (
        "n", "c", "h", "w", "kh", "kw", "sh", "sw", "pad_top", "pad_left", "dh", "dw", "ho", "wo",
        "layout", "c_stride", "dtype", "pad_")]


class Epilogue(C.Structure):
    _fields_ = [("bias", vp), ("residual", vp), ("alpha", f32), ("beta", f32),
                ("bias_mode", i32), ("act", i32), ("n_imm", i32), ("n_inst", i32),
                ("imm", f32 * 8), ("inst", EwInst * EW_MAX_INST), ("row_max", vp), ("row_max_ld", i64)]


class GemmArgs(C.Structure):
    _fields_ = [("a", vp), ("b", vp), ("out", vp), ("m", i64), ("n", i64), ("k", i64),
                ("lda", i64), ("ldb", i64), ("ldo", i64), ("batch", i64), ("stride_a", i64),
                ("stride_b", i64), ("stride_out", i64), ("stride_bias", i64), ("stride_res", i64),
                ("trans_a", i32), ("trans_b", i32), ("in_dtype", i32), ("out_dtype", i32),
                ("epi", Epilogue)]


class ConvArgs(C.Structure):
    _fields_ = [("x", vp), ("w", vp), ("out", vp)] + [(n, i32) for n in (
        "n", "c", "h", "w_", "c_stride", "c_pack", "o", "kh", "kw", "sh", "sw", "pad_top",
        "pad_left", "dh", "dw", "ho", "wo", "out_layout", "in_dtype", "out_dtype", "pad_")] + [
        ("epi", Epilogue)]


class AttnScoresArgs(C.Structure):
    _fields_ = [("q", vp), ("kt", vp), ("divisor", vp), ("mask", vp), ("out", vp)] + [
        (n, i32) for n in ("q0", "q1", "k0", "k1", "rows", "cols", "inner", "m0", "m1", "m2", "m3",
                           "in_dtype")]


class FlashArgs(C.Structure):
    _fields_ = [("q", vp), ("k", vp), ("v", vp), ("mask", vp), ("out", vp)] + [
        (n, i32) for n in ("batch", "heads", "seq_q", "seq_k", "head_dim", "dtype")] + [
        (n, i64) for n in ("q_sb", "q_sh", "q_ss", "k_sb", "k_sh", "k_ss", "v_sb", "v_sh", "v_ss",
                           "o_sb", "o_sh", "o_ss", "mask_ld")] + [("scale", f32), ("mask_kind", i32)]


class QuantizeArgs(C.Structure):
    _fields_ = [("x", vp), ("out", vp), ("count", i64), ("scale", f32), ("zero_point", i32),
                ("x_dtype", i32), ("pad_", i32)]


class QGemmArgs(C.Structure):
    _fields_ = [("a", vp), ("b", vp), ("out", vp), ("m", i64), ("n", i64), ("k", i64),
                ("lda", i64), ("ldb", i64), ("ldo", i64), ("a_zero", i32), ("b_zero", i32),
                ("a_scale", f32), ("y_scale", f32), ("b_scale", vp), ("y_zero", i32),
                ("mode", i32), ("out_dtype", i32), ("act_dtype", i32), ("q_scale", f32), ("q_zero", i32),
                ("epi", Epilogue)]


class DequantizeArgs(C.Structure):
    _fields_ = [("q", vp), ("out", vp), ("count", i64), ("scale", f32), ("zero_point", i32),
                ("out_dtype", i32), ("pad_", i32)]


class PackArgs(C.Structure):
    _fields_ = [("w", vp), ("out", vp)] + [(n, i32) for n in ("o", "c", "kh", "kw", "c_pack", "kw_pack")] + [
        ("k_stride", i64), ("in_dtype", i32), ("out_dtype", i32)]


class Fp8QuantArgs(C.Structure):
    _fields_ = [("x", vp), ("out", vp), ("scale", vp), ("rows", i64), ("cols", i64), ("ldx", i64),
                ("ldo", i64), ("x_dtype", i32), ("pad_", i32)]


class Fp8GemmArgs(C.Structure):
    _fields_ = [("a", vp), ("b", vp), ("a_scale", vp), ("b_scale", vp), ("out", vp), ("m", i64),
                ("n", i64), ("k", i64), ("lda", i64), ("ldb", i64), ("ldo", i64), ("out_dtype", i32),
                ("pad_", i32), ("epi", Epilogue)]


class Mxfp4QuantArgs(C.Structure):
    _fields_ = [("x", vp), ("codes", vp), ("scales", vp), ("rows", i64), ("cols", i64), ("ldx", i64),
                ("ldc", i64), ("lds", i64), ("x_dtype", i32), ("pad_", i32)]


class W4A16GemmArgs(C.Structure):
    _fields_ = [("a", vp), ("b_codes", vp), ("b_scales", vp), ("out", vp), ("m", i64), ("n", i64),
                ("k", i64), ("lda", i64), ("ldb", i64), ("ldbs", i64), ("ldo", i64), ("out_dtype", i32),
                ("pad_", i32), ("epi", Epilogue)]


class SplitKArgs(C.Structure):
    _fields_ = [("partial", vp), ("out", vp), ("m", i64), ("n", i64), ("ldo", i64), ("splits", i32),
                ("out_dtype", i32), ("epi", Epilogue)]


class ConvPoolArgs(C.Structure):
    _fields_ = [("x", vp), ("w", vp), ("bias", vp), ("out", vp)] + [(n, i32) for n in (
        "n", "c", "h", "w_", "o", "k_stride", "kh", "kw", "sh", "sw", "pad_top", "pad_left", "ho", "wo",
        "pkh", "pkw", "psh", "psw", "ppad_top", "ppad_left", "po", "qo", "relu", "in_dtype", "mm_dtype", "pad_")]


class Op(C.Structure):
    _fields_ = [("kind", i32), ("stream", i32), ("event", i32), ("pad_", i32), ("args", vp),
                ("dst", vp), ("src", vp), ("bytes", C.c_uint64)]


ABI_ORDER = [Props, FillArgs, CastArgs, EwArgs, CopyArgs, ReduceArgs, SoftmaxArgs, LayerNormArgs,
             BatchNormArgs, BnFoldArgs, GatherArgs, ArgmaxArgs, Im2colArgs, LayoutArgs, PoolArgs,
             Epilogue, GemmArgs, ConvArgs, AttnScoresArgs, FlashArgs, QuantizeArgs, QGemmArgs,
             DequantizeArgs, Op, PackArgs, ConvPoolArgs, Fp8QuantArgs, Fp8GemmArgs,
             SplitKArgs, Mxfp4QuantArgs, W4A16GemmArgs, ArgmaxFinishArgs, NonfiniteArgs]

# Kernel entry points: name -> args struct (all take (const args*, void* stream)).
KERNELS = {
    "c3h_fill": FillArgs, "c3h_cast": CastArgs, "c3h_ew": EwArgs, "c3h_strided_copy": CopyArgs,
    "c3h_reduce": ReduceArgs, "c3h_softmax": SoftmaxArgs, "c3h_layernorm": LayerNormArgs,
    "c3h_batchnorm": BatchNormArgs, "c3h_bn_fold": BnFoldArgs, "c3h_gather": GatherArgs,
    "c3h_argmax": ArgmaxArgs, "c3h_im2col": Im2colArgs, "c3h_layout": LayoutArgs,
    "c3h_maxpool2d": PoolArgs, "c3h_gemm": GemmArgs, "c3h_conv2d": ConvArgs,
    "c3h_attention_scores": AttnScoresArgs, "c3h_flash_attention": FlashArgs,
    "c3h_quantize": QuantizeArgs, "c3h_qgemm": QGemmArgs, "c3h_dequantize": DequantizeArgs,
    "c3h_pack_conv_weight": PackArgs, "c3h_conv_stem_pool": ConvPoolArgs,
    "c3h_quantize_fp8_rows": Fp8QuantArgs, "c3h_gemm_fp8": Fp8GemmArgs,
    "c3h_gemm_splitk_reduce": SplitKArgs, "c3h_quantize_mxfp4": Mxfp4QuantArgs,
    "c3h_gemm_w4a16": W4A16GemmArgs, "c3h_argmax_finish": ArgmaxFinishArgs, "c3h_nonfinite": NonfiniteArgs,
}

OP_KIND = {
    FillArgs: OP_FILL, CastArgs: OP_CAST, EwArgs: OP_EW, CopyArgs: OP_STRIDED_COPY,
    ReduceArgs: OP_REDUCE, SoftmaxArgs: OP_SOFTMAX, LayerNormArgs: OP_LAYERNORM,
    BatchNormArgs: OP_BATCHNORM, GatherArgs: OP_GATHER, ArgmaxArgs: OP_ARGMAX,
    Im2colArgs: OP_IM2COL, LayoutArgs: OP_LAYOUT, PoolArgs: OP_MAXPOOL, GemmArgs: OP_GEMM,
    ConvArgs: OP_CONV, AttnScoresArgs: OP_ATTN_SCORES, FlashArgs: OP_FLASH,
    QuantizeArgs: OP_QUANTIZE, QGemmArgs: OP_QGEMM, DequantizeArgs: OP_DEQUANTIZE,
    BnFoldArgs: OP_BNFOLD, PackArgs: OP_PACK, ConvPoolArgs: OP_CONV_POOL,
    Fp8QuantArgs: OP_QUANT_FP8, Fp8GemmArgs: OP_GEMM_FP8, SplitKArgs: OP_SPLITK,
    Mxfp4QuantArgs: OP_QUANT_MXFP4, W4A16GemmArgs: OP_GEMM_W4A16, ArgmaxFinishArgs: OP_ARGMAX_FINISH,
    NonfiniteArgs: OP_NONFINITE,
}

KERNEL_OF_ARGS = {v: k for k, v in KERNELS.items()}


class C3HError(RuntimeError):
    """A failed libc3hip.so call (status code and the library's message)."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(message)
        self.code = code


_LIB: Optional[C.CDLL] = None


def _declare(lib: C.CDLL) -> None:
    P = C.POINTER
    sig = {
        "c3h_init": ([C.c_int], C.c_int),
        "c3h_device_count": ([P(C.c_int)], C.c_int),
        "c3h_device_props": ([C.c_int, P(Props)], C.c_int),
        "c3h_last_error": ([], C.c_char_p),
        "c3h_device_synchronize": ([], C.c_int),
        "c3h_reload_switches": ([], C.c_int),
        "c3h_malloc": ([P(vp), C.c_size_t], C.c_int),
        "c3h_free": ([vp], C.c_int),
        "c3h_host_alloc": ([P(vp), C.c_size_t], C.c_int),
        "c3h_host_free": ([vp], C.c_int),
        "c3h_memcpy_h2d_async": ([vp, vp, C.c_size_t, vp], C.c_int),
        "c3h_memcpy_d2h_async": ([vp, vp, C.c_size_t, vp], C.c_int),
        "c3h_memcpy_d2d_async": ([vp, vp, C.c_size_t, vp], C.c_int),
        "c3h_memcpy_h2d": ([vp, vp, C.c_size_t], C.c_int),
        "c3h_memcpy_d2h": ([vp, vp, C.c_size_t], C.c_int),
        "c3h_stream_create": ([P(vp)], C.c_int),
        "c3h_stream_destroy": ([vp], C.c_int),
        "c3h_stream_synchronize": ([vp], C.c_int),
        "c3h_event_create": ([P(vp), C.c_int], C.c_int),
        "c3h_event_destroy": ([vp], C.c_int),
        "c3h_event_record": ([vp, vp], C.c_int),
        "c3h_stream_wait_event": ([vp, vp], C.c_int),
        "c3h_event_synchronize": ([vp], C.c_int),
        "c3h_event_elapsed_ms": ([P(C.c_float), vp, vp], C.c_int),
        "c3h_program_run": ([P(Op), i32, P(vp), i32, P(vp), i32], C.c_int),
        "c3h_program_capture": ([P(Op), i32, P(vp), i32, P(vp), i32, P(vp)], C.c_int),
        "c3h_graph_launch": ([vp, vp], C.c_int),
        "c3h_graph_destroy": ([vp], C.c_int),
        "c3h_abi_sizes": ([P(i64), i32], i32),
        "c3h_gemm_splitk": ([P(GemmArgs), i32, vp, C.c_size_t, vp], C.c_int),
        "c3h_gemm_splitk_noalloc": ([P(GemmArgs), i32, vp], C.c_int),
    }
    for name, (argtypes, restype) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    for name, struct in KERNELS.items():
        fn = getattr(lib, name)
        fn.argtypes = [P(struct), vp]
        fn.restype = C.c_int


def lib() -> C.CDLL:
    """Load libc3hip.so (built by `python -m hackathon_amd.build`)."""
    global _LIB
    if _LIB is None:
        path = Path(os.environ.get("C3HIP_LIB", str(LIB_PATH)))
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build it with `python -m hackathon_amd.build` "
                "(the HIP library is the only execution path)"
            )
        handle = C.CDLL(str(path))
        _declare(handle)
        _LIB = handle
        check_abi()
    return _LIB


def check_abi() -> None:
    """Compare ctypes struct sizes with the compiled library's sizeof()s."""
    handle = _LIB if _LIB is not None else lib()
    out = (i64 * 64)()
    n = handle.c3h_abi_sizes(out, 64)
    if n != len(ABI_ORDER):
        raise RuntimeError(f"ABI table length mismatch: library {n}, binding {len(ABI_ORDER)}")
    for i, struct in enumerate(ABI_ORDER):
        if C.sizeof(struct) != out[i]:
            raise RuntimeError(
                f"ABI mismatch for {struct.__name__}: ctypes {C.sizeof(struct)} bytes, "
                f"library {out[i]} bytes"
            )


def last_error() -> str:
    msg = lib().c3h_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(code: int, what: str = "") -> None:
    if code != 0:
        raise C3HError(code, f"{what or 'libc3hip'} failed ({code}): {last_error()}")


def call(name: str, args: C.Structure, stream: Optional[int] = None) -> None:
    """Invoke a kernel family entry point with its args struct."""
    fn = getattr(lib(), name)
    check(fn(C.byref(args), stream), name)


def launch(args: C.Structure, stream: Optional[int] = None) -> None:
    call(KERNEL_OF_ARGS[type(args)], args, stream)
