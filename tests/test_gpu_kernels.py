"""GPU checks of the kernel families the compiled path uses directly.

MFMA operand layouts, 16-bit GEMM, channels-last implicit-GEMM conv (fp32,
bf16, f16, narrow-channel stem), flash attention, layout conversion, and the
native timeline interpreter / hipGraph replay.  References are float64 NumPy
on the same (rounded) inputs; tolerances are stated per test.
"""

from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

import switches
from oracle import graph_ref as G
from oracle import registry_ref as R

pytestmark = pytest.mark.gpu


def _dev(x, dtype=None):
    from hackathon_amd.device import DeviceArray

    return DeviceArray.from_host(np.ascontiguousarray(x), dtype)


def _bits(x, kind):
    """Host array of 16-bit storage for kind in {'bf16','fp16'} + its float32 value."""
    from hackathon_amd.device import f32_to_bf16

    if kind == "bf16":
        bits = f32_to_bf16(x)
        return bits, G.round_bf16(x)
    h = np.asarray(x, np.float32).astype(np.float16)
    return h, h.astype(np.float32)


def _from16(arr, kind):
    from hackathon_amd.device import bf16_to_f32

    return bf16_to_f32(arr) if kind == "bf16" else np.asarray(arr).astype(np.float32)


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("m,n,k", [(16, 16, 32), (64, 64, 64), (300, 200, 96), (1000, 64, 576), (130, 600, 520),
                                   (77, 90, 136), (520, 1030, 1024)])
def test_gemm_16bit_matches_float64(gpu, kind, m, n, k):
    """16x16x32 MFMA operand layout + tiling: out = A @ B^T + bias, relu, fp32 out."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(m + n + k)
    a, af = _bits(rng.standard_normal((m, k), dtype=np.float32), kind)
    bt, bf = _bits(rng.standard_normal((n, k), dtype=np.float32), kind)
    bias = rng.standard_normal(n, dtype=np.float32)
    out = DeviceArray.empty((m, n), np.float32)
    code = _lib.BF16 if kind == "bf16" else _lib.F16
    bias_d = _dev(bias)  # kept alive until the launch completes: the epilogue holds a raw pointer
    E.gemm(_dev(a), _dev(bt), out, m, n, k, lda=k, ldb=k, ldo=n, trans_b=1, in_dtype=code,
           epi=E.epilogue(bias=bias_d, bias_mode=2, act=1))
    ref = np.maximum(af.astype(np.float64) @ bf.astype(np.float64).T + bias, 0)
    np.testing.assert_allclose(out.get(), ref, rtol=2e-5, atol=2e-4 * math.sqrt(k))


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("n", [260, 264])
def test_gemm_16bit_out_bias_residual_relu(gpu, kind, n):
    """16-bit output + per-column bias + residual + ReLU through the register
    epilogue: rows of 264 elements are 16-byte aligned (16-byte stores and
    residual loads, lane-swapped from the accumulator layout), rows of 260
    are not (8-byte form); both against float64 of the rounded operands."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(7 + n)
    m, k = 1000, 256
    a, af = _bits(rng.standard_normal((m, k), dtype=np.float32) * 0.5, kind)
    bt, bf = _bits(rng.standard_normal((n, k), dtype=np.float32) * 0.1, kind)
    res, resf = _bits(rng.standard_normal((m, n), dtype=np.float32), kind)
    bias = rng.standard_normal(n).astype(np.float32)
    code = _lib.BF16 if kind == "bf16" else _lib.F16
    out = DeviceArray.empty((m, n), a.dtype)
    ad, btd, resd, bd = _dev(a), _dev(bt), _dev(res), _dev(bias)
    out.copy_from_host(np.zeros((m, n), a.dtype))
    E.gemm(ad, btd, out, m, n, k, lda=k, ldb=k, ldo=n, trans_b=1, in_dtype=code,
           epi=E.epilogue(bias=bd, bias_mode=2, act=1, residual=resd))
    ref = np.maximum(af.astype(np.float64) @ bf.astype(np.float64).T + bias + resf, 0)
    got = _from16(out.get(), kind)
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=2e-2)
    assert np.count_nonzero(got) > got.size // 4


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_gemm_16bit_out_and_program_epilogue(gpu, kind):
    """16-bit output with a GELU program epilogue and a residual."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(1)
    m, n, k = 256, 192, 128
    a, af = _bits(rng.standard_normal((m, k), dtype=np.float32) * 0.5, kind)
    bt, bf = _bits(rng.standard_normal((n, k), dtype=np.float32) * 0.1, kind)
    res, resf = _bits(rng.standard_normal((m, n), dtype=np.float32), kind)
    code = _lib.BF16 if kind == "bf16" else _lib.F16
    out = DeviceArray.empty((m, n), a.dtype)
    # program: v/sqrt2 -> erf -> +1 -> x*() -> *0.5  (operands: 0=x, 1=prev, 2+j=imm[j])
    prog = [(_lib.EW_DIV, 0, 2, 0.0), (_lib.EW_ERF, 1, 1, 0.0), (_lib.EW_ADD, 1, 3, 0.0),
            (_lib.EW_MUL, 0, 1, 0.0), (_lib.EW_MUL, 1, 4, 0.0)]
    ad, btd, resd = _dev(a), _dev(bt), _dev(res)  # kept alive: the epilogue holds raw pointers
    E.gemm(ad, btd, out, m, n, k, lda=k, ldb=k, ldo=n, trans_b=1, in_dtype=code,
           epi=E.epilogue(residual=resd, program=prog, imm=[math.sqrt(2.0), 1.0, 0.5]))
    from scipy.special import erf
    v = af.astype(np.float64) @ bf.astype(np.float64).T + resf
    ref = 0.5 * v * (1 + erf(v / math.sqrt(2.0)))
    got = _from16(out.get(), kind)
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-2)
    # The compiled GELU activation (act 2; with these constants gelu_std)
    # follows the program's roundings with erf within about an fp32 step of
    # the correctly rounded one: the 16-bit results differ on at most 0.1 %
    # of elements, by one 16-bit step, or -- in the negative tail, where
    # both forms carry the chain's quantization of erf + 1 to 2^-24 and the
    # values are 16-bit subnormals -- by at most |x| 2^-22, the fp32 GELU
    # bound of test_gemm_gelu_epilogue_matches_the_chain.
    out2 = DeviceArray.empty((m, n), a.dtype)
    e2 = E.epilogue(residual=resd, imm=[math.sqrt(2.0), 1.0, 0.5])
    e2.act = 2
    E.gemm(ad, btd, out2, m, n, k, lda=k, ldb=k, ldo=n, trans_b=1, in_dtype=code, epi=e2)
    g2, g1 = out2.get(), out.get()
    step = np.abs(g2.view(np.int16).astype(np.int32) - g1.view(np.int16).astype(np.int32))
    d = np.abs(_from16(g2, kind).astype(np.float64) - _from16(g1, kind).astype(np.float64))
    ok = (step <= 1) | (d <= np.abs(v) * 2.0 ** -22)
    print(f"compiled GELU vs program ({kind}): {np.mean(step != 0):.2e} of elements differ, max {int(step.max())} "
          f"steps", flush=True)
    assert ok.all() and np.mean(step != 0) <= 1e-3, (int(step.max()), float(np.mean(step != 0)))


def _conv_case(rng, n, c, h, w, o, kh, kw, s, p):
    x = rng.standard_normal((n, c, h, w), dtype=np.float32)
    wt = rng.standard_normal((o, c, kh, kw), dtype=np.float32) * np.float32(math.sqrt(2.0 / (c * kh * kw)))
    b = rng.standard_normal(o, dtype=np.float32) * 0.1
    return x, wt, b, {"kernel_shape": [kh, kw], "strides": [s, s], "pads": [p, p, p, p], "dilations": [1, 1]}


@pytest.mark.parametrize("kind", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("case", [(2, 64, 14, 14, 64, 3, 3, 1, 1), (2, 64, 15, 15, 128, 3, 3, 2, 1),
                                  (2, 128, 8, 8, 256, 1, 1, 2, 0), (1, 3, 37, 37, 64, 7, 7, 2, 3),
                                  (3, 3, 16, 16, 64, 3, 3, 1, 1), (2, 40, 9, 9, 70, 3, 3, 1, 1),
                                  (1, 64, 12, 12, 64, 3, 3, 1, 2)])
def test_conv_nhwc_implicit_gemm(gpu, kind, case):
    """Channels-last implicit GEMM (+bias, +residual, relu) vs a float64 conv of the rounded operands."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(sum(case))
    n, c, h, w, o, kh, kw, s, p = case
    x, wt, b, attrs = _conv_case(rng, n, c, h, w, o, kh, kw, s, p)
    ho, wo = (h + 2 * p - kh) // s + 1, (w + 2 * p - kw) // s + 1
    code = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16}[kind]
    sdt = {"fp32": np.float32, "bf16": BF16, "fp16": np.float16}[kind]
    narrow = kind != "fp32" and c < 8
    c_pack = 4 if (kind == "fp32" or narrow) and c <= 4 else (c + 7) // 8 * 8 if kind != "fp32" else (c + 3) // 4 * 4
    kw_pack = ((kw + 7) // 8 * 8) if narrow else kw
    k = kh * kw_pack * c_pack
    k_stride = k if kind == "fp32" or narrow else (k + 31) // 32 * 32
    xd = E.to_nhwc(_dev(x), c_pack, out_dtype=sdt)
    wp = E.pack_conv_weight(_dev(wt), c_pack, kw_pack, k_stride, out_dtype=sdt)
    xr = x if kind == "fp32" else G.round_to(x, kind)
    wr = wt if kind == "fp32" else G.round_to(wt, kind)
    ref = R.conv2d(xr.astype(np.float64), wr.astype(np.float64), attrs).astype(np.float64) + b.reshape(1, o, 1, 1)
    resid = rng.standard_normal((n, ho, wo, o), dtype=np.float32)
    res_dev = _dev(resid) if kind == "fp32" else _dev(_bits(resid, kind)[0])
    ref = np.maximum(ref + (resid if kind == "fp32" else _bits(resid, kind)[1]).transpose(0, 3, 1, 2), 0)
    out = DeviceArray.empty((n, ho, wo, o), sdt)
    a = _lib.ConvArgs()
    a.x, a.w, a.out = xd.ptr, wp.ptr, out.ptr
    a.n, a.c, a.h, a.w_, a.c_stride, a.c_pack, a.o = n, c, h, w, c_pack, c_pack, o
    a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = kh, kw, s, s, p, p, 1, 1, ho, wo
    a.out_layout, a.in_dtype, a.out_dtype = 1, code, code
    b_dev = _dev(b)  # kept alive: the epilogue holds a raw pointer
    a.epi = E.epilogue(bias=b_dev, bias_mode=2, act=1, residual=res_dev)
    _lib.launch(a, None)
    got = out.get()
    got = got if kind == "fp32" else _from16(got, kind)
    tol = 1e-4 if kind == "fp32" else 2e-2
    np.testing.assert_allclose(got.transpose(0, 3, 1, 2), ref, rtol=tol, atol=tol)


@pytest.mark.parametrize("case", [(4, 32, 32, 64, 3, 1, 1, False, 1),    # the CIFAR ResNet's first conv (B = 4)
                                  (2, 15, 17, 16, 5, 2, 2, True, 0),
                                  (1, 37, 37, 64, 7, 2, 3, True, 1),     # 50 KB of weights in LDS
                                  (3, 9, 9, 32, 1, 1, 0, False, 0),
                                  (2, 11, 13, 256, 3, 2, 1, True, 1)])
def test_conv_direct_c4_matches_implicit_gemm(gpu, case):
    """fp32 conv of a 3-channel input (c_pack = c_stride = 4) on the direct VALU
    kernel: against the implicit-GEMM kernel (C3H_DISABLE_DIRECT_CONV) within
    fp32 summation-order differences, and against a float64 conv."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    n, h, w, o, k, s, p, with_res, act = case
    rng = np.random.default_rng(sum(case[:7]))
    x, wt, b, attrs = _conv_case(rng, n, 3, h, w, o, k, k, s, p)
    ho, wo = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    xd = E.to_nhwc(_dev(x), 4, out_dtype=np.float32)
    wp = E.pack_conv_weight(_dev(wt), 4, k, k * k * 4, out_dtype=np.float32)
    b_dev = _dev(b)
    resid = rng.standard_normal((n, ho, wo, o), dtype=np.float32)
    res_dev = _dev(resid) if with_res else None

    def run():
        out = DeviceArray.empty((n, ho, wo, o), np.float32)
        a = _lib.ConvArgs()
        a.x, a.w, a.out = xd.ptr, wp.ptr, out.ptr
        a.n, a.c, a.h, a.w_, a.c_stride, a.c_pack, a.o = n, 3, h, w, 4, 4, o
        a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = k, k, s, s, p, p, 1, 1, ho, wo
        a.out_layout, a.in_dtype, a.out_dtype = 1, _lib.F32, _lib.F32
        a.epi = E.epilogue(bias=b_dev, bias_mode=2, act=act, residual=res_dev)
        print(f"conv direct c4 case={case}", flush=True)
        _lib.launch(a, None)
        return out.get()

    got = run()
    gemm = switches.with_switch("C3H_DISABLE_DIRECT_CONV", "1", run)
    np.testing.assert_allclose(got, gemm, rtol=1e-5, atol=1e-5)
    ref = R.conv2d(x.astype(np.float64), wt.astype(np.float64), attrs) + b.reshape(1, o, 1, 1)
    if with_res:
        ref = ref + resid.transpose(0, 3, 1, 2)
    if act == 1:
        ref = np.maximum(ref, 0)
    np.testing.assert_allclose(got.transpose(0, 3, 1, 2), ref, rtol=1e-4, atol=1e-4)


def test_flash_attention_host_checks(gpu):
    """A head whose K (or V) rows span 2 GiB or more is refused before any
    launch: the kernel stages K and V with 32-bit buffer offsets."""
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    buf = DeviceArray.empty((4096,), np.uint16)
    a = _lib.FlashArgs()
    a.q = a.k = a.v = a.mask = a.out = buf.ptr
    a.batch, a.heads, a.seq_q, a.seq_k, a.head_dim, a.dtype = 1, 1, 16, 9, 64, _lib.F16
    a.q_sb = a.k_sb = a.v_sb = a.o_sb = 0
    a.q_sh = a.k_sh = a.v_sh = a.o_sh = 0
    a.q_ss = a.o_ss = 64
    a.k_ss, a.v_ss = 1 << 27, 64  # 8 rows x 2^27 elements x 2 bytes = 2 GiB
    a.mask_ld, a.scale, a.mask_kind = 0, 0.125, 0
    with pytest.raises(_lib.C3HError, match="2 GiB"):
        _lib.launch(a, None)
    a.k_ss, a.v_ss = 64, 1 << 27
    with pytest.raises(_lib.C3HError, match="2 GiB"):
        _lib.launch(a, None)


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("mask_kind", [0, 1, 2])
@pytest.mark.parametrize("b,h,s", [(2, 3, 64), (1, 2, 200), (2, 1, 256),
                                   (3, 5, 520)])  # 5 query tiles, 15 (batch, head) pairs, ragged key tile
def test_flash_attention(gpu, kind, mask_kind, b, h, s):
    """softmax(QK^T*scale + mask) V with Q,K,V head-split views of a packed [B,S,3,H,64] buffer.
    Blocks take the last query tiles of every (batch, head) first; the
    (3, 5, 520) case has a block count that is no multiple of 8 and several
    query tiles per head."""
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    d = 64
    rng = np.random.default_rng(b * 100 + h * 10 + s)
    qkv = rng.standard_normal((b, s, 3, h, d), dtype=np.float32)
    bits, val = _bits(qkv, kind)
    dev = _dev(bits)
    out = DeviceArray.empty((b, s, h, d), bits.dtype)  # written in [B,S,H,D] order
    mask = np.zeros((s, s), np.float32)
    if mask_kind == 2:
        mask = rng.standard_normal((s, s)).astype(np.float32)
        mask[np.triu_indices(s, 1)] = -np.inf
    mdev = _dev(mask)
    a = _lib.FlashArgs()
    item = 2
    base = dev.ptr
    a.q, a.k, a.v = base, base + h * d * item, base + 2 * h * d * item
    a.mask, a.out = mdev.ptr, out.ptr
    a.batch, a.heads, a.seq_q, a.seq_k, a.head_dim = b, h, s, s, d
    a.dtype = _lib.BF16 if kind == "bf16" else _lib.F16
    sb, ss, sh = s * 3 * h * d, 3 * h * d, d
    a.q_sb = a.k_sb = a.v_sb = sb
    a.q_sh = a.k_sh = a.v_sh = sh
    a.q_ss = a.k_ss = a.v_ss = ss
    a.o_sb, a.o_sh, a.o_ss = s * h * d, d, h * d
    a.mask_ld, a.scale, a.mask_kind = s, 1.0 / math.sqrt(d), mask_kind
    _lib.launch(a, None)
    got = _from16(out.get(), kind).transpose(0, 2, 1, 3)
    q, k, v = (val[:, :, i].transpose(0, 2, 1, 3).astype(np.float64) for i in range(3))
    sc = q @ k.transpose(0, 1, 3, 2) / math.sqrt(d)
    if mask_kind == 1:
        sc = sc + np.triu(np.full((s, s), -np.inf), 1)
    elif mask_kind == 2:
        sc = sc + mask
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = p @ v
    tol = 2e-2 if kind == "bf16" else 5e-3
    np.testing.assert_allclose(got, ref, rtol=tol, atol=tol)


@pytest.mark.parametrize("c,c_pad,kind,hw", [(3, 4, "bf16", (9, 13)), (64, 64, "fp32", (9, 13)),
                                             (40, 48, "fp16", (9, 13)), (3, 8, "fp32", (9, 13)),
                                             (3, 4, "bf16", (8, 12)), (3, 4, "fp32", (6, 6)), (1, 4, "fp16", (4, 5))])
def test_layout_roundtrip(gpu, c, c_pad, kind, hw):
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    h, w = hw
    x = np.random.default_rng(c).standard_normal((2, c, h, w)).astype(np.float32)
    sdt = {"fp32": np.float32, "bf16": BF16, "fp16": np.float16}[kind]
    nhwc = E.to_nhwc(_dev(x), c_pad, out_dtype=sdt)
    host = nhwc.get()
    val = host if kind == "fp32" else _from16(host, kind)
    xr = x if kind == "fp32" else G.round_to(x, kind)
    np.testing.assert_array_equal(val[..., :c], xr.transpose(0, 2, 3, 1))
    np.testing.assert_array_equal(val[..., c:], 0)
    back = DeviceArray.empty(x.shape, np.float32)
    a = _lib.LayoutArgs()
    a.in_, a.out, a.n, a.c, a.h, a.w = nhwc.ptr, back.ptr, 2, c, h, w
    a.c_pad, a.direction, a.in_dtype, a.out_dtype = c_pad, 1, nhwc.code, _lib.F32
    _lib.launch(a, None)
    np.testing.assert_array_equal(back.get(), xr)


def test_program_run_and_graph_replay(gpu):
    """The native timeline interpreter and a captured hipGraph replayed 5 times."""
    import ctypes as C

    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray, Stream, synchronize

    x = np.linspace(-1, 1, 4096, dtype=np.float32)
    xd = _dev(x)
    y = DeviceArray.empty((4096,), np.float32)
    z = DeviceArray.empty((4096,), np.float32)
    fill = _lib.FillArgs(out=z.ptr, count=4096, dtype=_lib.F32, value=0.0)
    ew1 = E.ew_args([xd], [(_lib.EW_RELU, 0, 0, 0.0)], y, (4096,))
    ew2 = E.ew_args([y, xd], [(_lib.EW_ADD, 0, 1, 0.0), (_lib.EW_MUL_IMM, 2, 2, 3.0)], z, (4096,))
    ops = (_lib.Op * 3)()
    for i, args in enumerate([fill, ew1, ew2]):
        ops[i].kind = _lib.OP_KIND[type(args)]
        ops[i].stream = 0
        ops[i].args = C.cast(C.pointer(args), C.c_void_p)
    s = Stream()
    streams = (C.c_void_p * 1)(s.handle)
    _lib.check(_lib.lib().c3h_program_run(ops, 3, streams, 1, None, 0), "program_run")
    s.synchronize()
    expect = (np.maximum(x, 0) + x) * 3
    np.testing.assert_allclose(z.get(), expect, rtol=1e-6)
    g = C.c_void_p()
    _lib.check(_lib.lib().c3h_program_capture(ops, 3, streams, 1, None, 0, C.byref(g)), "capture")
    for _ in range(5):
        xd.copy_from_host(np.zeros(4096, np.float32))
        synchronize()
        np.testing.assert_array_equal(z.get(), expect)  # untouched until replay
        _lib.check(_lib.lib().c3h_graph_launch(g, s.handle), "graph_launch")
        s.synchronize()
        np.testing.assert_array_equal(z.get(), 0)
        xd.copy_from_host(x)
        _lib.check(_lib.lib().c3h_graph_launch(g, s.handle), "graph_launch")
        s.synchronize()
        np.testing.assert_allclose(z.get(), expect, rtol=1e-6)
    _lib.check(_lib.lib().c3h_graph_destroy(g), "graph_destroy")


@pytest.mark.parametrize("mode,n,out_kind", [(2, 200, "fp32"), (3, 200, "fp32"), (3, 200, "bf16"), (3, 70, "fp32"),
                                              (2, 96, "fp16"), (2, 260, "bf16"), (3, 196, "fp16"), (3, 264, "bf16")])
def test_qgemm_fused_dequant_epilogue_bit_exact(gpu, mode, n, out_kind):
    """Modes 2/3 (dequantize / QLinearMatMul->DequantizeLinear) + bias + residual + relu, float32 order.
    16-bit rows of 8k + 4 elements (n = 260, 196) take the interior epilogue's
    8-byte stores and residual loads, 16-byte aligned ones (n = 200, 264)
    the 16-byte form."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(mode * 1000 + n)
    m, k = 300, 256
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    bt = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa, sy = np.float32(0.02), np.float32(0.37)
    sb = (rng.random(n) * 0.01 + 0.001).astype(np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    res32 = rng.standard_normal((m, n), dtype=np.float32)
    acc = (a.astype(np.int64) @ bt.T.astype(np.int64)).astype(np.int32)
    if mode == 3:
        v = R.requantize(acc, sa, sb, sy, 0).astype(np.float32) * sy
    else:
        v = acc.astype(np.float32) * (sa * sb)
    code, sdt = {"fp32": (_lib.F32, np.float32), "bf16": (_lib.BF16, BF16), "fp16": (_lib.F16, np.float16)}[out_kind]
    if out_kind == "fp32":
        res_dev, res_used = _dev(res32), res32
    else:
        bits, res_used = _bits(res32, out_kind)
        res_dev = _dev(bits)
    want = np.maximum((v + bias) + res_used, 0).astype(np.float32)
    out = DeviceArray.empty((m, n), sdt)
    g = _lib.QGemmArgs()
    ad, bd, sbd, biasd = _dev(a), _dev(bt), _dev(sb), _dev(bias)
    g.a, g.b, g.out, g.m, g.n, g.k, g.lda, g.ldb, g.ldo = ad.ptr, bd.ptr, out.ptr, m, n, k, k, k, n
    g.a_scale, g.y_scale, g.b_scale, g.mode, g.out_dtype = sa, sy, sbd.ptr, mode, code
    g.epi = E.epilogue(bias=biasd, bias_mode=2, act=1, residual=res_dev)
    _lib.launch(g, None)
    got = out.get()
    if out_kind == "fp32":
        np.testing.assert_array_equal(got, want)
    else:
        np.testing.assert_array_equal(_from16(got, out_kind), G.round_to(want, out_kind))


@pytest.mark.parametrize("kind", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("c,c_stride,geom", [(64, 64, (3, 2, 1)), (16, 24, (3, 2, 1)), (8, 8, (2, 2, 0)), (6, 6, (3, 1, 1))])
def test_maxpool_nhwc(gpu, kind, c, c_stride, geom):
    """Channels-last max pool (vector and scalar paths) vs the oracle on the rounded input."""
    from hackathon_amd import _lib
    from hackathon_amd.device import BF16, DeviceArray

    k, st, pd = geom
    rng = np.random.default_rng(c + k)
    n, h, w = 2, 15, 14
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    xr = x if kind == "fp32" else G.round_to(x, kind)
    attrs = {"kernel_shape": [k, k], "strides": [st, st], "pads": [pd] * 4}
    ref = R.maxpool2d(xr, attrs)
    ho, wo = ref.shape[2:]
    store = np.zeros((n, h, w, c_stride), np.float32)
    store[..., :c] = x.transpose(0, 2, 3, 1)
    sdt = {"fp32": np.float32, "bf16": BF16, "fp16": np.float16}[kind]
    xd = _dev(store) if kind == "fp32" else _dev(_bits(store, kind)[0])
    out = DeviceArray.empty((n, ho, wo, c_stride), sdt)
    a = _lib.PoolArgs()
    a.x, a.out, a.n, a.c, a.h, a.w = xd.ptr, out.ptr, n, c, h, w
    a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw = k, k, st, st, pd, pd, 1, 1
    a.ho, a.wo, a.layout, a.c_stride = ho, wo, 1, c_stride
    a.dtype = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16}[kind]
    _lib.launch(a, None)
    got = out.get()
    got = got if kind == "fp32" else _from16(got, kind)
    np.testing.assert_array_equal(got[..., :c].transpose(0, 3, 1, 2), ref)


@pytest.mark.parametrize("kind,out_kind", [("fp32", "fp32"), ("bf16", "bf16"), ("fp16", "fp16"), ("bf16", "fp32")])
@pytest.mark.parametrize("cols,residual", [(512, False), (768, True), (72, True), (4096, False), (100, False)])
def test_layernorm_vectorized_and_fallback(gpu, kind, out_kind, cols, residual):
    """Row LayerNorm (+residual) in fp32 statistics vs the oracle on the rounded inputs."""
    from hackathon_amd import _lib
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(cols)
    rows = 37
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 3 + 1
    r = rng.standard_normal((rows, cols)).astype(np.float32)
    g = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    code = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16}
    sdt = {"fp32": np.float32, "bf16": BF16, "fp16": np.float16}
    if kind == "fp32":
        xd, rd, xr, rr = _dev(x), _dev(r), x, r
    else:
        (xb, xr), (rb, rr) = _bits(x, kind), _bits(r, kind)
        xd, rd = _dev(xb), _dev(rb)
    gd, bd = _dev(g), _dev(b)
    out = DeviceArray.empty((rows, cols), sdt[out_kind])
    a = _lib.LayerNormArgs()
    a.x, a.residual, a.scale, a.bias, a.out = xd.ptr, rd.ptr if residual else None, gd.ptr, bd.ptr, out.ptr
    a.rows, a.cols, a.epsilon, a.x_dtype, a.out_dtype = rows, cols, 1e-5, code[kind], code[out_kind]
    _lib.launch(a, None)
    got = out.get()
    got = got if out_kind == "fp32" else _from16(got, out_kind)
    want = R.layer_norm((xr + rr) if residual else xr, g, b, -1, 1e-5)[0]
    tol = 2e-5 if out_kind == "fp32" else (2e-2 if out_kind == "bf16" else 4e-3)
    np.testing.assert_allclose(got, want, rtol=tol, atol=tol * 4)


@pytest.mark.parametrize("kind", ["fp32", "bf16", "fp16"])
def test_quantize_vectorized_bit_exact(gpu, kind):
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(3)
    x = (rng.standard_normal(4096 * 3) * 40).astype(np.float32)
    x[:6] = [0.5, 1.5, 2.5, -0.5, 1000.0, -1000.0]
    xr = x if kind == "fp32" else _bits(x, kind)[1]
    xd = _dev(x) if kind == "fp32" else _dev(_bits(x, kind)[0])
    out = DeviceArray.empty(x.shape, np.int8)
    a = _lib.QuantizeArgs()
    a.x, a.out, a.count, a.scale, a.zero_point = xd.ptr, out.ptr, x.size, 0.5, 0
    a.x_dtype = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16}[kind]
    _lib.launch(a, None)
    np.testing.assert_array_equal(out.get(), R.quantize(xr, np.float32(0.5), 0))


def _f32(bits):
    return np.array([bits], np.uint32).view(np.float32)[0]


# Scales for the division-free quantizer: all-ones significands (the divisors
# where a reciprocal-only quotient is most often misrounded), tiny and huge
# exponents (the quotient is formed from x 2^-e), the smallest normal scale.
_QUANT_SCALES = [0.5, 0.019, 1 / 127, 0.0123, 3.0, 40.11176,
                 _f32(0x3FFFFFFF), _f32(0x3F7FFFFF), _f32(0x3C7FFFFF),     # 2 - 2^-22, 1 - 2^-24, 2^-6 (2 - 2^-23)
                 _f32(0x0D800000), _f32(0x0D7FFFFF),                        # 2^-100 and just below
                 _f32(0x71800000), _f32(0x71800001),                        # 2^100 and just above
                 1e-30, 7e30, _f32(0x00800000), _f32(0x7F7FFFFF)]           # 2^-126, the largest float


@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("zero", [0, -3, 5])
def test_quantize_every_code_boundary_bit_exact(gpu, kind, zero):
    """c3h_quantize (vectorized and scalar kernels) equals rne(x / scale) with a
    correctly rounded fp32 division, for every finite and infinite bf16 / fp16
    value, and for fp32 values within a few ulps of every half-integer
    quotient (the rounding boundaries of the codes), over the scales above."""
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    code = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16}[kind]
    for scale in _QUANT_SCALES:
        s = np.float32(scale)
        if kind == "bf16":
            bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
            xr = (bits.astype(np.uint32) << 16).view(np.float32)
            keep = ~np.isnan(xr)
            bits, xr = bits[keep], xr[keep]
            host = bits
        elif kind == "fp16":
            h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
            h = h[~np.isnan(h)]
            host, xr = h, h.astype(np.float32)
        else:
            k = np.arange(-140.5, 140.0, 1.0)                      # half-integer quotients around every code
            near = [(k * np.float64(s)).astype(np.float32)]
            for _ in range(2):                                     # and 1, 2 ulps either side
                near = [np.nextafter(near[0], np.float32(-np.inf))] + near + [np.nextafter(near[-1], np.float32(np.inf))]
            specials = np.array([np.inf, -np.inf, 0.0, -0.0, 3e38, -3e38, 1e-40, -1e-40], np.float32)
            xr = np.concatenate(near + [specials]).astype(np.float32)
            xr = xr[~np.isnan(xr)]
            host = xr
        want = R.quantize(xr, s, zero)
        for count in (xr.size - xr.size % 8, xr.size - xr.size % 8 - 1):   # vectorized, then the scalar kernel
            xd = _dev(np.ascontiguousarray(host[:count]))
            out = DeviceArray.empty((count,), np.int8)
            a = _lib.QuantizeArgs()
            a.x, a.out, a.count, a.scale, a.zero_point, a.x_dtype = xd.ptr, out.ptr, count, float(s), zero, code
            print(f"quantize {kind} scale={float(s)!r} zero={zero} count={count}", flush=True)
            _lib.launch(a, None)
            got = out.get()
            bad = np.nonzero(got != want[:count])[0]
            assert bad.size == 0, (float(s), xr[bad[:5]], got[bad[:5]], want[:count][bad[:5]])


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("n,h,w,relu,in_kind", [(2, 64, 64, 1, "fp32"), (3, 70, 57, 1, "fp32"), (1, 45, 83, 0, "fp32"),
                                                (2, 38, 40, 1, "same"), (2, 224, 224, 1, "fp32"),
                                                (1, 100, 60, 0, "same"), (1, 61, 92, 1, "fp32"),
                                                (2, 64, 64, 1, "fp32 nonfinite"), (2, 64, 64, 0, "fp32 nonfinite")])
def test_conv_stem_pool_matches_unfused_chain(gpu, kind, n, h, w, relu, in_kind):
    """c3h_conv_stem_pool == layout -> c3h_conv2d (bias, relu) -> c3h_maxpool2d, bit for bit;
    and within 16-bit rounding of a float64 conv + max pool of the rounded operands.

    The fused kernel pools the raw accumulators before bias, ReLU and rounding; the
    "nonfinite" cases put NaN and +-inf inputs in (NaN and +-inf conv values, whole
    windows of NaN, inf - inf) so that the NaN rules of the two orders are compared too."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(h * w + n)
    x, wt, b, attrs = _conv_case(rng, n, 3, h, w, 64, 7, 7, 2, 3)
    nonfinite = in_kind.endswith("nonfinite")
    if nonfinite:
        in_kind = "fp32"
        x[0, 0, 10:12, 10:12] = np.nan  # conv rows / columns 4-7 NaN: pooled (3, 3) sees only NaN
        for (i, c, r, q), v in {(0, 1, 30, 40): np.inf, (1, 2, 50, 5): -np.inf, (1, 0, 33, 33): np.inf,
                                (1, 1, 34, 35): -np.inf, (0, 0, 0, 63): np.nan, (1, 2, 63, 0): np.inf}.items():
            x[i, c, r, q] = v
    code = {"bf16": _lib.BF16, "fp16": _lib.F16}[kind]
    sdt = {"bf16": BF16, "fp16": np.float16}[kind]
    ho, wo = (h + 6 - 7) // 2 + 1, (w + 6 - 7) // 2 + 1
    po, qo = (ho + 2 - 3) // 2 + 1, (wo + 2 - 3) // 2 + 1
    xd = _dev(x) if in_kind == "fp32" else _dev(_bits(x, kind)[0])
    wp = E.pack_conv_weight(_dev(wt), 4, 8, 224, out_dtype=sdt)
    bd = _dev(b)
    # unfused chain through the C ABI
    xn = E.to_nhwc(xd, 4, out_dtype=sdt)
    conv = DeviceArray.empty((n, ho, wo, 64), sdt)
    a = _lib.ConvArgs()
    a.x, a.w, a.out = xn.ptr, wp.ptr, conv.ptr
    a.n, a.c, a.h, a.w_, a.c_stride, a.c_pack, a.o = n, 3, h, w, 4, 4, 64
    a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = 7, 7, 2, 2, 3, 3, 1, 1, ho, wo
    a.out_layout, a.in_dtype, a.out_dtype = 1, code, code
    a.epi = E.epilogue(bias=bd, bias_mode=2, act=relu)
    _lib.launch(a, None)
    pooled = DeviceArray.empty((n, po, qo, 64), sdt)
    pa = _lib.PoolArgs()
    pa.x, pa.out, pa.n, pa.c, pa.h, pa.w = conv.ptr, pooled.ptr, n, 64, ho, wo
    pa.kh, pa.kw, pa.sh, pa.sw, pa.pad_top, pa.pad_left, pa.dh, pa.dw = 3, 3, 2, 2, 1, 1, 1, 1
    pa.ho, pa.wo, pa.layout, pa.c_stride, pa.dtype = po, qo, 1, 64, code
    _lib.launch(pa, None)
    # fused
    fused = DeviceArray.empty((n, po, qo, 64), sdt)
    f = _lib.ConvPoolArgs()
    f.x, f.w, f.bias, f.out = xd.ptr, wp.ptr, bd.ptr, fused.ptr
    f.n, f.c, f.h, f.w_, f.o, f.k_stride = n, 3, h, w, 64, 224
    f.kh, f.kw, f.sh, f.sw, f.pad_top, f.pad_left, f.ho, f.wo = 7, 7, 2, 2, 3, 3, ho, wo
    f.pkh, f.pkw, f.psh, f.psw, f.ppad_top, f.ppad_left, f.po, f.qo = 3, 3, 2, 2, 1, 1, po, qo
    f.relu, f.in_dtype, f.mm_dtype = relu, _lib.F32 if in_kind == "fp32" else code, code
    print(f"conv_stem_pool {kind} n={n} {h}x{w} relu={relu} in={in_kind}", flush=True)
    _lib.launch(f, None)
    got = fused.get()
    np.testing.assert_array_equal(got.view(np.uint16), pooled.get().view(np.uint16))
    if nonfinite:
        g = _from16(got, kind)
        assert not np.isnan(g).any() and (g == np.inf).any()
        assert (g[0, 3, 3] == (0.0 if relu else -np.inf)).all()
        return
    xr, wr = G.round_to(x, kind), G.round_to(wt, kind)
    ref = R.conv2d(xr.astype(np.float64), wr.astype(np.float64), attrs) + b.reshape(1, 64, 1, 1)
    ref = np.maximum(ref, 0) if relu else ref
    ref = R.maxpool2d(ref.astype(np.float32), {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]})
    np.testing.assert_allclose(_from16(got, kind).transpose(0, 3, 1, 2), ref, rtol=1e-2, atol=1e-2)


def test_conv_stem_pool_rejects_other_geometry(gpu):
    from hackathon_amd import _lib

    f = _lib.ConvPoolArgs()
    f.x = f.w = f.out = 16
    f.n, f.c, f.h, f.w_, f.o, f.k_stride = 1, 3, 32, 32, 64, 224
    f.kh, f.kw, f.sh, f.sw, f.pad_top, f.pad_left, f.ho, f.wo = 5, 5, 2, 2, 2, 2, 16, 16
    f.pkh, f.pkw, f.psh, f.psw, f.ppad_top, f.ppad_left, f.po, f.qo = 3, 3, 2, 2, 1, 1, 8, 8
    f.mm_dtype, f.in_dtype = _lib.BF16, _lib.F32
    with pytest.raises(_lib.C3HError, match="7x7"):
        _lib.launch(f, None)


def test_bf16_narrowing_is_round_to_nearest_even_bit_exact(gpu):
    """fp32 -> bf16 (the hardware conversion every 16-bit epilogue uses) equals the integer
    round-to-nearest-even formula on ties, denormals, infinities, NaN payloads and random patterns."""
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray, f32_to_bf16

    special = np.array([0x3F808000, 0x3F818000, 0x3F80FFFF, 0x00000001, 0x007FFFFF, 0x00008000, 0x00018000,
                        0x7F800000, 0xFF800000, 0x7F7FFFFF, 0x7F7F8000, 0x80000000, 0x7F800001, 0xFFC00001,
                        0x7FFFFFFF, 0x7FBFFFFF, 0x807F8000], np.uint32)
    rnd = np.random.default_rng(11).integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    bits = np.concatenate([special, rnd])
    x = DeviceArray.from_host(bits.view(np.float32))
    out = DeviceArray.empty(x.shape, BF16)
    E.cast_into(x, out)
    np.testing.assert_array_equal(out.get().view(np.uint16), f32_to_bf16(bits.view(np.float32)).view(np.uint16))


@pytest.mark.parametrize("out_kind", ["fp32", "bf16", "fp16"])
def test_splitk_reduce_fixed_order_bit_exact(gpu, out_kind):
    """c3h_gemm_splitk_reduce: partials summed in split order, then alpha,
    beta * bias, residual and ReLU in the common epilogue's float32 order."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(7)
    splits, m, n = 7, 130, 70
    part = rng.standard_normal((splits, m, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    r32 = rng.standard_normal((m, n)).astype(np.float32)
    code, sdt = {"fp32": (_lib.F32, np.float32), "bf16": (_lib.BF16, BF16), "fp16": (_lib.F16, np.float16)}[out_kind]
    if out_kind == "fp32":
        res_dev, res_val = _dev(r32), r32
    else:
        bits, res_val = _bits(r32, out_kind)
        res_dev = _dev(bits)
    acc = part[0].copy()
    for s_ in range(1, splits):
        acc = (acc + part[s_]).astype(np.float32)
    want = np.maximum(((np.float32(0.5) * acc) + np.float32(2.0) * bias[None, :]) + res_val, 0).astype(np.float32)
    out = DeviceArray.empty((m, n), sdt)
    pd, bd = _dev(part), _dev(bias)
    g = _lib.SplitKArgs()
    g.partial, g.out, g.m, g.n, g.ldo, g.splits, g.out_dtype = pd.ptr, out.ptr, m, n, n, splits, code
    g.epi = E.epilogue(bias=bd, bias_mode=2, alpha=0.5, beta=2.0, act=1, residual=res_dev)
    _lib.launch(g, None)
    got = out.get()
    if out_kind == "fp32":
        np.testing.assert_array_equal(got, want)
    else:
        np.testing.assert_array_equal(_from16(got, out_kind), G.round_to(want, out_kind))


@pytest.mark.parametrize("kind_name,dt", [("fp32", "fp32"), ("bf16", "bf16"), ("fp16", "fp16")])
@pytest.mark.parametrize("outer,red,inner", [(3, 49, 512), (2, 13, 8), (5, 3, 1024), (1, 64, 136), (256, 16, 512),
                                             (256, 49, 512), (2, 65, 256), (3, 200, 64)])
def test_reduce_channels_last_vec(gpu, kind_name, dt, outer, red, inner):
    """Channels-last reductions (inner % 8 == 0: GlobalAveragePool over NHWC;
    reduce <= 64 on the 16-position-group kernel, longer on the four-wave
    one): max exact, sum / mean within float32 summation error of float64."""
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(outer * 100 + red + inner)
    x32 = rng.standard_normal((outer, red, inner)).astype(np.float32)
    if dt == "fp32":
        xd, xv, code = _dev(x32), x32, _lib.F32
    else:
        bits, xv = _bits(x32, dt)
        xd, code = _dev(bits), (_lib.BF16 if dt == "bf16" else _lib.F16)
    for kind in (0, 1, 2):
        out = DeviceArray.empty((outer, inner), np.float32)
        a = _lib.ReduceArgs()
        a.in_, a.out, a.outer, a.reduce, a.inner = xd.ptr, out.ptr, outer, red, inner
        a.kind, a.in_dtype, a.out_dtype = kind, code, _lib.F32
        _lib.launch(a, None)
        got = out.get()
        x64 = xv.astype(np.float64)
        if kind == 0:
            np.testing.assert_array_equal(got, xv.max(axis=1))
        else:
            want = x64.sum(axis=1) / (red if kind == 2 else 1)
            bound = np.abs(x64).sum(axis=1) / (red if kind == 2 else 1) * red * 2.0 ** -23
            assert np.all(np.abs(got - want) <= bound + 1e-7)


@pytest.mark.parametrize("rows,cols,res,bias,dt", [(37, 512, False, True, "fp16"), (16384 // 64, 512, True, True, "fp16"),
                                                  (5, 1024, True, False, "bf16"), (7, 2048, False, True, "fp32"),
                                                  (3, 4096, True, True, "fp16"), (1, 8, False, False, "fp32")])
def test_layernorm_vec_against_float64(gpu, rows, cols, res, bias, dt):
    """Vectorized LayerNorm (one wave per row, 1-8 vectors per lane): mean,
    centred variance and the affine map against float64 of the same inputs."""
    from hackathon_amd import _lib
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(rows + cols)
    x32 = (rng.standard_normal((rows, cols)) * 3 + 1).astype(np.float32)
    r32 = rng.standard_normal((rows, cols)).astype(np.float32)
    g = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    if dt == "fp32":
        xd, xv, rd, rv, code, sdt = _dev(x32), x32, _dev(r32), r32, _lib.F32, np.float32
    else:
        xb, xv = _bits(x32, dt)
        rb, rv = _bits(r32, dt)
        xd, rd = _dev(xb), _dev(rb)
        code, sdt = (_lib.BF16, BF16) if dt == "bf16" else (_lib.F16, np.float16)
    out = DeviceArray.empty((rows, cols), sdt)
    mean_d, inv_d = DeviceArray.empty((rows,), np.float32), DeviceArray.empty((rows,), np.float32)
    gd, bd = _dev(g), _dev(b)
    a = _lib.LayerNormArgs()
    a.x, a.residual, a.scale, a.bias, a.out = xd.ptr, rd.ptr if res else None, gd.ptr, bd.ptr if bias else None, out.ptr
    a.mean_out, a.invstd_out, a.rows, a.cols, a.epsilon = mean_d.ptr, inv_d.ptr, rows, cols, 1e-5
    a.x_dtype, a.out_dtype = code, code
    print(f"layernorm rows={rows} cols={cols} res={res} bias={bias} {dt}", flush=True)
    _lib.launch(a, None)
    s = (xv.astype(np.float64) + (rv if res else 0))
    mu = s.mean(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(((s - mu) ** 2).mean(axis=1, keepdims=True) + 1e-5)
    want = (s - mu) * inv * g + (b if bias else 0)
    got = out.get()
    got = got.astype(np.float32) if dt != "bf16" else _from16(got, "bf16")
    tol = {"fp32": 1e-4, "fp16": 2e-3, "bf16": 1.6e-2}[dt]
    np.testing.assert_allclose(got, want, rtol=tol, atol=tol * 4)
    np.testing.assert_allclose(mean_d.get(), mu[:, 0], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(inv_d.get(), inv[:, 0], rtol=1e-4)


def _bigtile_pair(launch):
    """Run `launch` with the eight-wave kernels (256x256, 256x192) allowed, then with them disabled."""
    a = _with_env("C3H_DISABLE_BIGTILE", None, launch)
    b = _with_env("C3H_DISABLE_BIGTILE", "1", launch)
    return a, b


@pytest.mark.parametrize("kind,out_kind,act,m,n,k", [
    ("bf16", "bf16", 1, 4096, 4096, 192), ("fp16", "fp32", 1, 4096, 4096, 192), ("fp16", "fp16", 2, 4096, 4096, 192),
    ("fp16", "fp16", 1, 16384, 1536, 512),   # the fp16 decoder's QKV: the 256x192 kernel
    ("fp16", "fp16", 2, 8192, 1536, 256),    # 256x192 with GELU in registers
])
def test_gemm_big_tile_matches_128_tiles(gpu, kind, out_kind, act, m, n, k):
    """Shapes with enough tiles that an eight-wave kernel is chosen (256x256;
    256x192 for fp16 output with N a multiple of 192), with bias + residual +
    ReLU or GELU (computed in registers there, through the staged epilogue by
    the 128x128 kernel): bit-identical to the 128x128 kernel (same K order
    per output and the same epilogue arithmetic) and within the 16-bit GEMM
    tolerance of float64 on sampled rows."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(11 + n)
    a32 = (rng.standard_normal((m, k)) * 0.5).astype(np.float32)
    b32 = (rng.standard_normal((n, k)) * 0.5).astype(np.float32)
    ab, av = _bits(a32, kind)
    bb, bv = _bits(b32, kind)
    bias = rng.standard_normal(n).astype(np.float32)
    r32 = rng.standard_normal((m, n)).astype(np.float32)
    code = _lib.BF16 if kind == "bf16" else _lib.F16
    ocode, sdt = {"fp32": (_lib.F32, np.float32), "bf16": (_lib.BF16, BF16), "fp16": (_lib.F16, np.float16)}[out_kind]
    if out_kind == "fp32":
        rd, rv = _dev(r32), r32
    else:
        rb, rv = _bits(r32, out_kind)
        rd = _dev(rb)
    ad, bd, biasd = _dev(ab), _dev(bb), _dev(bias)
    out = DeviceArray.empty((m, n), sdt)

    def launch():
        g = _lib.GemmArgs()
        g.a, g.b, g.out = ad.ptr, bd.ptr, out.ptr
        g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = m, n, k, k, k, n, 1
        g.trans_a, g.trans_b, g.in_dtype, g.out_dtype = 0, 1, code, ocode
        g.epi = E.epilogue(bias=biasd, bias_mode=2, act=act, residual=rd,
                           imm=[math.sqrt(2.0), 1.0, 0.5] if act == 2 else [])
        print(f"gemm {m}x{n}x{k} {kind}->{out_kind} act={act}", flush=True)
        _lib.launch(g, None)
        return out.get().copy()
    big, small = _bigtile_pair(launch)
    np.testing.assert_array_equal(big.view(np.uint8), small.view(np.uint8))
    rows = np.arange(0, m, 97)
    t = av[rows].astype(np.float64) @ bv.astype(np.float64).T + bias + rv[rows]
    if act == 1:
        want = np.maximum(t, 0)
    else:
        from scipy.special import erf

        want = t * (erf(t / math.sqrt(2.0)) + 1.0) * 0.5
    got = big[rows] if out_kind == "fp32" else _from16(big[rows], out_kind)
    tol = 1e-4 if out_kind == "fp32" else 1e-2
    np.testing.assert_allclose(got, want, rtol=tol, atol=tol * 4)


@pytest.mark.parametrize("c0,c1,c2", [(math.sqrt(2.0), 1.0, 0.5),   # the standard constants: gelu_std
                                      (1.5, 1.0, 0.5)])            # others: the chain form, gelu_erf
def test_gemm_gelu_epilogue_matches_the_chain(gpu, c0, c1, c2):
    """The GEMM GELU epilogue (act 2) on exact accumulators x (A = [x, 0, 0, 0],
    B row 0 = 1): equal to the decomposed chain ((x * (erf(x / c0) + c1)) *
    c2) evaluated in fp32 with a correctly rounded erf, within 2^-21 relative
    plus |x| 2^-22 (two fp32 steps of erf near +-1, where the chain's own
    rounding of erf dominates), over [-12, 12] and the special values."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray
    from scipy.special import erf

    x = np.concatenate([np.linspace(-12, 12, 48000, dtype=np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 1e-8, -1e-8, 3.0, -3.0, np.inf, -np.inf, np.nan],
                                 np.float32)])
    m = ((x.size + 63) // 64) * 64
    a = np.zeros((m, 4), np.float32)
    a[: x.size, 0] = x
    n = 16
    b = np.zeros((4, n), np.float32)
    b[0] = 1.0
    ad, bd = _dev(a), _dev(b)
    out = DeviceArray.empty((m, n), np.float32)
    g = _lib.GemmArgs()
    g.a, g.b, g.out = ad.ptr, bd.ptr, out.ptr
    g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = m, n, 4, 4, n, n, 1
    g.trans_a, g.trans_b, g.in_dtype, g.out_dtype = 0, 0, _lib.F32, _lib.F32
    g.epi = E.epilogue(act=2, imm=[c0, c1, c2])
    print(f"gemm fp32 gelu epilogue m={m} constants {c0, c1, c2}", flush=True)
    _lib.launch(g, None)
    got = out.get()[: x.size]
    np.testing.assert_array_equal(got, np.repeat(got[:, :1], n, axis=1))
    got = got[:, 0].astype(np.float64)
    f = np.float32
    q = (x / f(c0)).astype(f)
    e = erf(q.astype(np.float64)).astype(f)
    with np.errstate(invalid="ignore"):
        ref = ((x * (e + f(c1))).astype(f) * f(c2)).astype(f).astype(np.float64)
    fin = np.isfinite(ref)
    tol = 2.0 ** -21 * np.abs(ref[fin]) + np.abs(x[fin].astype(np.float64)) * 2.0 ** -22 + 1e-38
    err = np.abs(got[fin] - ref[fin])
    assert np.all(err <= tol), (float(np.max(err / tol)), float(x[fin][np.argmax(err / tol)]))
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    assert got[np.isposinf(x)][0] == np.inf


@pytest.mark.parametrize("n,c,h,w,o,stride,resid", [
    # (each case is large enough for the host to pick the 256x256 tile: its
    # rounds of resident tiles beat 128x128's by 10 %)
    (256, 256, 14, 14, 256, 1, False),   # ResNet-18 224 layer 3 (36 K tiles)
    (200, 256, 14, 14, 256, 1, True),    # ragged M (153.1 tiles of 256 rows), residual
    (200, 128, 28, 28, 256, 2, False),   # a stride-2 downsampling 3x3 (18 K tiles)
    (500, 512, 7, 7, 384, 1, True),      # N = 1.5 tiles, 72 K tiles, ragged M
])
def test_conv_big_tile_matches_128_tiles(gpu, n, c, h, w, o, stride, resid):
    """3x3 convs with N > 128 take the 256x256 kernel with the ping-pong
    schedule; bit-identical to the same tile without it (C3H_DISABLE_PP) and
    to the 128x128 kernel, and a float64 spot check."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(12 + n + o)
    ho, wo = (h + 2 - 3) // stride + 1, (w + 2 - 3) // stride + 1
    x32 = rng.standard_normal((n, h, w, c)).astype(np.float32)
    w32 = (rng.standard_normal((o, 3, 3, c)) * 0.05).astype(np.float32)
    xb, xv = _bits(x32, "bf16")
    wb, wv = _bits(w32.reshape(o, -1), "bf16")
    rb, rv = _bits(rng.standard_normal((n, ho, wo, o)).astype(np.float32), "bf16")
    bias = rng.standard_normal(o).astype(np.float32)
    xd, wd, bd, rd = _dev(xb), _dev(wb), _dev(bias), _dev(rb)
    out = DeviceArray.empty((n, ho, wo, o), BF16)

    def launch():
        a = _lib.ConvArgs()
        a.x, a.w, a.out = xd.ptr, wd.ptr, out.ptr
        a.n, a.c, a.h, a.w_, a.c_stride, a.c_pack, a.o = n, c, h, w, c, c, o
        a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = 3, 3, stride, stride, 1, 1, 1, 1, ho, wo
        a.out_layout, a.in_dtype, a.out_dtype = 1, _lib.BF16, _lib.BF16
        a.epi = E.epilogue(bias=bd, bias_mode=2, act=1, residual=rd if resid else None)
        print(f"conv n={n} {c}->{o} {h}x{w}/{stride} resid={resid} 3x3 bf16", flush=True)
        out.copy_from_host(np.zeros((n, ho, wo, o), np.uint16))
        _lib.launch(a, None)
        return out.get().copy()
    big, small = _bigtile_pair(launch)
    plain = _with_env("C3H_DISABLE_PP", "1", launch)
    np.testing.assert_array_equal(big.view(np.uint16), small.view(np.uint16))
    np.testing.assert_array_equal(big.view(np.uint16), plain.view(np.uint16))
    got = _from16(big, "bf16")
    xp = np.pad(xv.astype(np.float64), ((0, 0), (1, 1), (1, 1), (0, 0)))
    wv4 = wv.astype(np.float64).reshape(o, 3, 3, c)
    for (b_, y, x_) in [(0, 0, 0), (n // 3, ho // 2, wo - 1), (n - 1, ho - 1, wo // 2), (n // 2, ho // 2, ho // 2)]:
        patch = xp[b_, stride * y:stride * y + 3, stride * x_:stride * x_ + 3, :]
        want = np.einsum("hwc,ohwc->o", patch, wv4) + bias + (rv[b_, y, x_] if resid else 0.0)
        np.testing.assert_allclose(got[b_, y, x_], np.maximum(want, 0), rtol=1e-2, atol=4e-2)


@pytest.mark.parametrize("n,c,h,w,o,ksz,stride,resid,dt,out_dt", [
    (256, 128, 28, 28, 128, 3, 1, True, "bf16", "bf16"),   # ResNet-18 224 layer 2 (1255 tiles of 160 rows)
    (256, 64, 56, 56, 128, 3, 2, False, "bf16", "bf16"),   # its stride-2 entry conv
    (256, 64, 56, 56, 128, 1, 2, False, "bf16", "bf16"),   # its 1x1 downsampling shortcut
    (200, 128, 28, 28, 128, 3, 1, True, "fp16", "f32"),    # ragged M (980 tiles), fp16 in, fp32 out
    (203, 128, 28, 28, 128, 3, 1, False, "bf16", "bf16"),  # ragged last tile (159152 rows)
])
def test_conv_tile160_matches_128_tiles(gpu, n, c, h, w, o, ksz, stride, resid, dt, out_dt):
    """16-bit implicit-GEMM convs whose 160 x 128 tiles fill fewer rounds of
    the chip than 128 x 128 ones take the 160-row kernel: bit-identical to the
    128 x 128 kernel (C3H_DISABLE_TILE160; same K order per element), and a
    float64 spot check."""
    m = n * ((h + 2 * (ksz // 2) - ksz) // stride + 1) * ((w + 2 * (ksz // 2) - ksz) // stride + 1)
    # the host's choice for a 256-CU device: 160-row rounds cost 1.25 rounds of 128 x 128
    r128 = -(-(-(-m // 128) * -(-o // 128)) // 512)
    r160 = -(-(-(-m // 160) * (o // 128)) // 512) * 1.25
    assert r160 < 0.97 * r128, (r160, r128)
    _conv_alt_tile_check(n, c, h, w, o, ksz, stride, resid, dt, out_dt, ["C3H_DISABLE_TILE160"])


def _conv_alt_tile_check(n, c, h, w, o, ksz, stride, resid, dt, out_dt, switches_off):
    """Runs a conv with the default kernel choice and with each switch in
    switches_off set; all outputs bit-identical; float64 spot check."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    pad = ksz // 2
    ho, wo = (h + 2 * pad - ksz) // stride + 1, (w + 2 * pad - ksz) // stride + 1
    rng = np.random.default_rng(31 + n + o + ksz)
    x32 = rng.standard_normal((n, h, w, c)).astype(np.float32)
    w32 = (rng.standard_normal((o, ksz, ksz, c)) * 0.05).astype(np.float32)
    xb, xv = _bits(x32, dt)
    wb, wv = _bits(w32.reshape(o, -1), dt)
    r32 = rng.standard_normal((n, ho, wo, o)).astype(np.float32)
    if out_dt == "f32":
        rb, rv = r32, r32
    else:
        rb, rv = _bits(r32, out_dt)
    bias = rng.standard_normal(o).astype(np.float32)
    xd, wd, bd, rd = _dev(xb), _dev(wb), _dev(bias), _dev(rb)
    out = DeviceArray.empty((n, ho, wo, o), np.float32 if out_dt == "f32" else BF16)
    in_code = _lib.BF16 if dt == "bf16" else _lib.F16
    out_code = _lib.F32 if out_dt == "f32" else _lib.BF16

    def launch():
        a = _lib.ConvArgs()
        a.x, a.w, a.out = xd.ptr, wd.ptr, out.ptr
        a.n, a.c, a.h, a.w_, a.c_stride, a.c_pack, a.o = n, c, h, w, c, c, o
        a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = (
            ksz, ksz, stride, stride, pad, pad, 1, 1, ho, wo)
        a.out_layout, a.in_dtype, a.out_dtype = 1, in_code, out_code
        a.epi = E.epilogue(bias=bd, bias_mode=2, act=1, residual=rd if resid else None)
        print(f"conv n={n} {c}->{o} {h}x{w} k{ksz}/{stride} resid={resid} {dt}->{out_dt}", flush=True)
        out.copy_from_host(np.zeros(out.nbytes, np.uint8))
        _lib.launch(a, None)
        return out.get().copy()
    got_default = launch()
    view = np.uint32 if out_dt == "f32" else np.uint16
    for var in switches_off:
        other = _with_env(var, "1", launch)
        np.testing.assert_array_equal(got_default.view(view), other.view(view), err_msg=var)
    got = got_default if out_dt == "f32" else _from16(got_default, out_dt)
    assert np.any(got != 0)
    xp = np.pad(xv.astype(np.float64), ((0, 0), (pad, pad), (pad, pad), (0, 0)))
    wv4 = wv.astype(np.float64).reshape(o, ksz, ksz, c)
    for (b_, y, x_) in [(0, 0, 0), (n // 3, ho // 2, wo - 1), (n - 1, ho - 1, wo - 1), (n // 2, ho // 2, ho // 2)]:
        patch = xp[b_, stride * y:stride * y + ksz, stride * x_:stride * x_ + ksz, :]
        want = np.einsum("hwc,ohwc->o", patch, wv4) + bias + (rv[b_, y, x_] if resid else 0.0)
        np.testing.assert_allclose(got[b_, y, x_], np.maximum(want, 0), rtol=1e-2, atol=4e-2)


@pytest.mark.parametrize("m,n,k,mode,act", [
    (4096, 4096, 256, 0, 0), (4096, 4096, 256, 2, 0), (4096, 4096, 256, 3, 2),
    # N a multiple of 192 with bf16 output: the 256x192 kernel
    (16384, 768, 768, 2, 0),      # the W8A8 out projection (bias + residual)
    (4096, 2304, 256, 3, 2),      # QKV-shaped, GELU in registers
    (16000, 768, 256, 3, 0),      # ragged M (16000 = 62.5 tiles): edge tiles
])
def test_qgemm_big_tile_matches_128_tiles(gpu, m, n, k, mode, act):
    """int8 GEMM on the eight-wave kernels (256x256; 256x192 where N is a
    multiple of 192 and the output bf16): int32 accumulators (mode 0) equal
    the exact integer product; the dequantized bf16 output with bias +
    residual (mode 2), and requantize -> dequantize + bias + GELU (mode 3,
    computed in registers there and through the staged epilogue by the
    128x128 kernel) are bit-identical to the 128x128 kernel."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(13 + mode + n)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    bt = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sb = (rng.random(n) * 0.01 + 0.001).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    rb, _ = _bits(rng.standard_normal((m, n)).astype(np.float32), "bf16")
    ad, bd, sbd, biasd, rd = _dev(a), _dev(bt), _dev(sb), _dev(bias), _dev(rb)
    out = DeviceArray.empty((m, n), np.int32 if mode == 0 else BF16)

    def launch():
        g = _lib.QGemmArgs()
        g.a, g.b, g.out, g.m, g.n, g.k, g.lda, g.ldb, g.ldo = ad.ptr, bd.ptr, out.ptr, m, n, k, k, k, n
        g.a_scale, g.y_scale, g.b_scale, g.mode = 0.02, 0.37, sbd.ptr, mode
        g.out_dtype = _lib.I32 if mode == 0 else _lib.BF16
        if mode == 2:
            g.epi = E.epilogue(bias=biasd, bias_mode=2, residual=rd)
        elif mode == 3:
            g.epi = E.epilogue(bias=biasd, bias_mode=2, act=act, imm=[math.sqrt(2.0), 1.0, 0.5])
        else:
            g.epi = E.epilogue()
        out.copy_from_host(np.zeros(out.nbytes, np.uint8))  # a launch that writes nothing cannot pass
        print(f"qgemm {m}x{n}x{k} mode {mode} act {act}", flush=True)
        _lib.launch(g, None)
        return out.get().copy()
    big, small = _bigtile_pair(launch)
    np.testing.assert_array_equal(big.view(np.uint8), small.view(np.uint8))
    assert np.any(big.view(np.uint8) != 0)
    if mode == 0:
        rows = np.arange(0, m, 61)
        np.testing.assert_array_equal(big[rows], a[rows].astype(np.int64) @ bt.T.astype(np.int64))


@pytest.mark.parametrize("m,n,k,mode,act,act_kind,switch,qscale", [
    (4096, 4096, 256, 3, 2, "bf16", None, 0.0417),                  # 256x256 tile, GELU in registers
    (4096, 4096, 256, 3, 2, "bf16", "C3H_DISABLE_BIGTILE", 0.0417), # 128x128 DMA tile, staged GELU epilogue
    (300, 200, 256, 3, 1, "fp16", None, 0.0417),                    # 128x128, direct epilogue
    (300, 70, 256, 2, 0, "fp32", None, 0.0417),                     # unaligned rows: staged, partial stores
    (300, 200, 256, 3, 2, "bf16", "C3H_DISABLE_DMA", 0.0417),       # register-prefetch kernel
    (16384, 3072, 768, 3, 2, "bf16", None, 0.0417),                 # W8A8 FFN1
    (4096, 4096, 256, 2, 1, "bf16", None, 0.06),                    # multiplier fp32(1 / 0.06) - 1 ulp
    (4096, 4096, 256, 3, 2, "bf16", "C3H_DISABLE_QMUL", 0.0417),    # division form in the interior tiles too
])
def test_qgemm_int8_output_equals_qgemm_then_quantize(gpu, m, n, k, mode, act, act_kind, switch, qscale):
    """Modes 2 / 3 with an int8 output (the QuantizeLinear after the epilogue
    in the same launch) give exactly the codes of the two-launch form: the
    float epilogue stored in act_kind, then c3h_quantize -- with saturated
    codes and a nonzero zero point.  The interior tiles of a bf16 activation
    quantize with one multiply by a multiplier the host checked against the
    division over all 65536 bf16 values: fp32(1 / q_scale) for 0.0417, its
    neighbour 1 ulp below for 0.06 (where x / 0.06 sits on a rounding tie
    for some x and fp32(1 / 0.06) rounds those the other way)."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(m + n + k + act)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    bt = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sb = (rng.random(n) * 0.01 + 0.001).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    ad, bd, sbd, biasd = _dev(a), _dev(bt), _dev(sb), _dev(bias)
    code, sdt = {"fp32": (_lib.F32, np.float32), "bf16": (_lib.BF16, BF16), "fp16": (_lib.F16, np.float16)}[act_kind]
    qzero = 3
    mid = DeviceArray.empty((m, n), sdt)
    want = DeviceArray.empty((m, n), np.int8)
    got = DeviceArray.empty((m, n), np.int8)

    def qgemm(out, out_code, quant):
        g = _lib.QGemmArgs()
        g.a, g.b, g.out, g.m, g.n, g.k, g.lda, g.ldb, g.ldo = ad.ptr, bd.ptr, out.ptr, m, n, k, k, k, n
        g.a_scale, g.y_scale, g.b_scale, g.mode, g.out_dtype = 0.02, 0.37, sbd.ptr, mode, out_code
        if quant:
            g.act_dtype, g.q_scale, g.q_zero = code, qscale, qzero
        g.epi = E.epilogue(bias=biasd, bias_mode=2, act=act, imm=[math.sqrt(2.0), 1.0, 0.5] if act == 2 else [])
        print(f"qgemm {m}x{n}x{k} mode {mode} act {act} {act_kind} quant={quant} switch={switch}", flush=True)
        _lib.launch(g, None)

    def run():
        qgemm(mid, code, False)
        q = _lib.QuantizeArgs()
        q.x, q.out, q.count, q.scale, q.zero_point, q.x_dtype = mid.ptr, want.ptr, m * n, qscale, qzero, code
        _lib.launch(q, None)
        got.copy_from_host(np.full(m * n, 77, np.int8))
        qgemm(got, _lib.I8, True)
        return want.get(), got.get()

    w, g_ = _with_env(switch, "1", run) if switch else run()
    bad = np.argwhere(w != g_)
    assert bad.size == 0, (bad[:5], w[tuple(bad[:5].T)], g_[tuple(bad[:5].T)])
    assert (w == 127).any() and (act != 0 or (w == -128).any()) and len(np.unique(w)) > 50


def test_qgemm_int8_output_host_checks(gpu):
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    a = DeviceArray.empty((32, 64), np.int8)
    out = DeviceArray.empty((32, 32), np.int8)
    sb = DeviceArray.empty((32,), np.float32)
    g = _lib.QGemmArgs()
    g.a, g.b, g.out, g.m, g.n, g.k, g.lda, g.ldb, g.ldo = a.ptr, a.ptr, out.ptr, 32, 32, 64, 64, 64, 32
    g.a_scale, g.y_scale, g.b_scale, g.mode, g.out_dtype = 0.02, 0.37, sb.ptr, 3, _lib.I8
    g.act_dtype, g.q_scale, g.q_zero = _lib.BF16, 0.0, 0
    g.epi = E.epilogue()
    with pytest.raises(_lib.C3HError, match="q_scale"):
        _lib.launch(g, None)
    g.q_scale, g.act_dtype = 0.5, _lib.I32
    with pytest.raises(_lib.C3HError, match="act_dtype"):
        _lib.launch(g, None)
    g.act_dtype = _lib.BF16
    g.epi = E.epilogue(residual=out)
    with pytest.raises(_lib.C3HError, match="residual"):
        _lib.launch(g, None)


def test_gemm_fp8_big_tile_matches_128_tiles(gpu):
    """E4M3 GEMM 4096x4096x512 on the 256x256 kernel: bit-identical to the
    128x128 kernel (same K order), integer operands exact."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    from oracle import fp8_ref as F8

    rng = np.random.default_rng(14)
    m = n = 4096
    k = 512
    vals = np.arange(-8, 9, dtype=np.float32)
    qa, qb = F8.encode(rng.choice(vals, (m, k))), F8.encode(rng.choice(vals, (n, k)))
    sa, sb = np.ones(m, np.float32), np.ones(n, np.float32)
    keep = [_dev(qa), _dev(qb), _dev(sa), _dev(sb)]
    out = DeviceArray.empty((m, n), np.float32)

    def launch():
        g = _lib.Fp8GemmArgs()
        g.a, g.b, g.a_scale, g.b_scale, g.out = keep[0].ptr, keep[1].ptr, keep[2].ptr, keep[3].ptr, out.ptr
        g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.out_dtype = m, n, k, k, k, n, _lib.F32
        g.epi = E.epilogue()
        print(f"gemm_fp8 {m}x{n}x{k}", flush=True)
        _lib.launch(g, None)
        return out.get().copy()
    big, small = _bigtile_pair(launch)
    np.testing.assert_array_equal(big, small)
    rows = np.arange(0, m, 61)
    np.testing.assert_array_equal(big[rows], (F8.decode(qa[rows]).astype(np.float64) @ F8.decode(qb).astype(np.float64).T).astype(np.float32))


@pytest.mark.parametrize("kind,n,h,w,resid,act,bias", [
    ("bf16", 256, 56, 56, True, 1, True),    # ResNet-18 224 layer 1, second conv of a block
    ("bf16", 256, 56, 56, False, 1, True),   # first conv of a block
    ("fp16", 3, 13, 10, True, 1, True),      # ragged last band (13 rows, 11 per band)
    ("bf16", 2, 9, 62, False, 0, False),     # wide rows, no bias, no ReLU
    ("fp16", 1, 1, 5, True, 0, True),        # one output row
    ("bf16", 5, 20, 70, True, 1, True),      # one-row bands (70 wide)
    ("bf16", 2, 6, 100, True, 1, False),     # too wide for a band: generic path on both sides
])
def test_conv3x3_band_kernel_matches_implicit_gemm(gpu, kind, n, h, w, resid, act, bias):
    """The banded 3x3 / 64-channel kernel (conv3x3.hip) against the generic
    implicit-GEMM path (C3H_DISABLE_CONV3X3) on the same inputs: bit-identical
    (same K order and epilogue arithmetic), output zero-filled before each
    run; plus a float64 spot check of the rounded operands."""
    import os

    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(n * 1000 + h * 10 + w)
    c = o = 64
    x32 = rng.standard_normal((n, h, w, c)).astype(np.float32)
    w32 = (rng.standard_normal((o, 3, 3, c)) * 0.06).astype(np.float32)
    xb, xv = _bits(x32, kind)
    wb, wv = _bits(w32.reshape(o, -1), kind)
    b32 = rng.standard_normal(o).astype(np.float32)
    r32 = rng.standard_normal((n, h, w, o)).astype(np.float32)
    rb, rv = _bits(r32, kind)
    code, sdt = (_lib.BF16, BF16) if kind == "bf16" else (_lib.F16, np.float16)
    xd, wd, bd, rd = _dev(xb), _dev(wb), _dev(b32), _dev(rb)
    out = DeviceArray.empty((n, h, w, o), sdt)
    zeros = np.zeros((n, h, w, o), dtype=np.uint16)

    def launch(disable):
        out.copy_from_host(zeros)
        a = _lib.ConvArgs()
        a.x, a.w, a.out = xd.ptr, wd.ptr, out.ptr
        a.n, a.c, a.h, a.w_, a.c_stride, a.c_pack, a.o = n, c, h, w, c, c, o
        a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = 3, 3, 1, 1, 1, 1, 1, 1, h, w
        a.out_layout, a.in_dtype, a.out_dtype = 1, code, code
        a.epi = E.epilogue(bias=bd if bias else None, bias_mode=2 if bias else 0, act=act,
                           residual=rd if resid else None)
        def go():
            print(f"conv3x3 {kind} n={n} h={h} w={w} resid={resid} act={act} bias={bias} generic={disable}", flush=True)
            _lib.launch(a, None)
            return out.get().copy()

        return _with_env("C3H_DISABLE_CONV3X3", "1" if disable else None, go)

    band = launch(False)
    generic = launch(True)
    np.testing.assert_array_equal(band.view(np.uint16), generic.view(np.uint16))
    got = _from16(band, kind)
    xp = np.pad(xv.astype(np.float64), ((0, 0), (1, 1), (1, 1), (0, 0)))
    wv4 = wv.astype(np.float64).reshape(o, 3, 3, c)
    for (b_, y, x_) in [(0, 0, 0), (n - 1, h - 1, w - 1), (n // 2, h // 2, w // 3), (0, h - 1, 0)]:
        t = np.einsum("hwc,ohwc->o", xp[b_, y:y + 3, x_:x_ + 3, :], wv4)
        t = t + (b32 if bias else 0) + (rv[b_, y, x_] if resid else 0)
        want = np.maximum(t, 0) if act == 1 else t
        np.testing.assert_allclose(got[b_, y, x_], want, rtol=1e-2, atol=4e-2)


@pytest.mark.parametrize("kind", ["fp16", "bf16"])
@pytest.mark.parametrize("mask_kind", [1, 2])
def test_flash_attention_config5_shape(gpu, kind, mask_kind):
    """Flash attention at the W8A8 decoder's shape: B=16, H=12, S=1024, dh=64,
    causal (computed) or additive (causal -inf plus random finite values).
    Every (batch, head) is checked against float64 at 40 query rows (tile
    edges, the first and last rows, random rows), and one whole (b, h) at every
    row, so a wrong batch/head/tile offset anywhere in the grid fails."""
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    b, h, s, d = 16, 12, 1024, 64
    rng = np.random.default_rng(1024 + mask_kind)
    qkv = rng.standard_normal((b, s, 3, h, d), dtype=np.float32)
    bits, val = _bits(qkv, kind)
    del qkv
    dev = _dev(bits)
    out = DeviceArray.empty((b, s, h, d), bits.dtype)
    mask = np.zeros((s, s), np.float32)
    if mask_kind == 2:
        mask = rng.standard_normal((s, s)).astype(np.float32)
        mask[np.triu_indices(s, 1)] = -np.inf
    mdev = _dev(mask)
    a = _lib.FlashArgs()
    item = 2
    a.q, a.k, a.v = dev.ptr, dev.ptr + h * d * item, dev.ptr + 2 * h * d * item
    a.mask, a.out = mdev.ptr, out.ptr
    a.batch, a.heads, a.seq_q, a.seq_k, a.head_dim = b, h, s, s, d
    a.dtype = _lib.BF16 if kind == "bf16" else _lib.F16
    a.q_sb = a.k_sb = a.v_sb = s * 3 * h * d
    a.q_sh = a.k_sh = a.v_sh = d
    a.q_ss = a.k_ss = a.v_ss = 3 * h * d
    a.o_sb, a.o_sh, a.o_ss = s * h * d, d, h * d
    a.mask_ld, a.scale, a.mask_kind = s, 1.0 / math.sqrt(d), mask_kind
    print(f"flash B={b} H={h} S={s} {kind} mask_kind={mask_kind}", flush=True)
    _lib.launch(a, None)
    got = _from16(out.get(), kind)  # [B, S, H, D]
    add = np.triu(np.full((s, s), -np.inf), 1) if mask_kind == 1 else mask.astype(np.float64)

    def ref_rows(bi, hi, rows):
        q = val[bi, rows, 0, hi].astype(np.float64)
        k = val[bi, :, 1, hi].astype(np.float64)
        v = val[bi, :, 2, hi].astype(np.float64)
        sc = q @ k.T / math.sqrt(d) + add[rows]
        p = np.exp(sc - sc.max(-1, keepdims=True))
        return (p / p.sum(-1, keepdims=True)) @ v

    rows = np.unique(np.concatenate([[0, 1, 15, 16, 31, 63, 64, 65, 127, 128, 129, 255, 256, 511, 512, 767, 768,
                                      1000, 1022, 1023], rng.integers(0, s, 20)]))
    tol = 2e-2 if kind == "bf16" else 5e-3
    worst = 0.0
    for bi in range(b):
        for hi in range(h):
            want = ref_rows(bi, hi, rows)
            err = np.abs(got[bi, rows, hi] - want)
            worst = max(worst, float(err.max()))
            np.testing.assert_allclose(got[bi, rows, hi], want, rtol=tol, atol=tol)
    full = ref_rows(b - 1, h - 1, np.arange(s))
    np.testing.assert_allclose(got[b - 1, :, h - 1], full, rtol=tol, atol=tol)
    print(f"  max |err| at sampled rows {worst:.3e}, whole (b,h)=({b - 1},{h - 1}) "
          f"{float(np.abs(got[b - 1, :, h - 1] - full).max()):.3e}", flush=True)


@pytest.mark.parametrize("kind,addend", [("fp32", "fp32"), ("bf16", "bf16"), ("fp16", "fp16"), ("bf16", "fp32"),
                                          ("fp16", "fp32")])
@pytest.mark.parametrize("n_idx,rows,inner", [(64 * 256, 256, 512), (16 * 1024, 1024, 768), (37, 5, 8)])
def test_gather_fused_addend_bit_exact(gpu, kind, addend, n_idx, rows, inner):
    """c3h_gather with an addend: out[r] = data[idx[r]] + addend[r % rows],
    fp32 add of the stored values and one rounding -- what Gather followed by
    the broadcast Add gives -- including negative indices; the decoder
    embedding shapes of configs 4 and 5 and a ragged small case.  With an
    fp32 addend and 16-bit data (the compiled decoders' form) the table is
    not rounded before the add: the unfused 16-bit Gather then the Add of the
    fp32 table, bit for bit."""
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(n_idx + inner)
    vocab = 300
    table = rng.standard_normal((vocab, inner)).astype(np.float32)
    pos = rng.standard_normal((rows, inner)).astype(np.float32)
    idx = rng.integers(-vocab, vocab, size=n_idx).astype(np.int64)
    if kind == "fp32":
        t_st, t_val, code = table, table, _lib.F32
    else:
        t_st, t_val = _bits(table, kind)
        code = _lib.BF16 if kind == "bf16" else _lib.F16
    if addend == "fp32":
        p_st, p_val, acode = pos, pos, _lib.F32
    else:
        (p_st, p_val), acode = _bits(pos, addend), code
    want = t_val[idx] + p_val[np.arange(n_idx) % rows]
    want = want if kind == "fp32" else G.round_to(want, kind)
    td, pd, idd = _dev(t_st), _dev(p_st), _dev(idx)
    out = DeviceArray.empty((n_idx, inner), t_st.dtype)
    flag = _dev(np.zeros(1, np.int32))
    a = _lib.GatherArgs()
    a.data, a.indices, a.out, a.error_flag = td.ptr, idd.ptr, out.ptr, flag.ptr
    a.outer, a.axis_dim, a.inner, a.n_indices, a.elem_bytes = 1, vocab, inner, n_idx, t_st.itemsize
    a.dtype, a.addend, a.addend_rows, a.addend_dtype = code, pd.ptr, rows, acode
    _lib.launch(a, None)
    got = out.get() if kind == "fp32" else _from16(out.get(), kind)
    np.testing.assert_array_equal(got, want)
    assert int(flag.get()[0]) == 0
    if addend == "fp32" and kind != "fp32":
        # the table really enters unrounded: rounding it first changes some outputs
        pre = G.round_to(t_val[idx] + G.round_to(pos, kind)[np.arange(n_idx) % rows], kind)
        assert n_idx < 100 or not np.array_equal(pre, want)


def test_gather_out_of_range_sets_flag_and_zero_rows(gpu):
    """An index outside [-axis_dim, axis_dim) writes a zero row and sets the
    error flag (plain and fused-addend forms); in-range rows are unaffected."""
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    table = np.arange(10 * 8, dtype=np.float32).reshape(10, 8) + 1.0
    idx = np.array([0, 9, 10, -11, -10, 3], np.int64)
    for fused in (False, True):
        td, idd = _dev(table), _dev(idx)
        pos = _dev(np.zeros((2, 8), np.float32))
        out = DeviceArray.empty((6, 8), np.float32)
        flag = _dev(np.zeros(1, np.int32))
        a = _lib.GatherArgs()
        a.data, a.indices, a.out, a.error_flag = td.ptr, idd.ptr, out.ptr, flag.ptr
        a.outer, a.axis_dim, a.inner, a.n_indices, a.elem_bytes = 1, 10, 8, 6, 4
        if fused:
            a.dtype, a.addend, a.addend_rows, a.addend_dtype = _lib.F32, pos.ptr, 2, _lib.F32
        _lib.launch(a, None)
        got = out.get()
        assert int(flag.get()[0]) == 1
        np.testing.assert_array_equal(got[[0, 1, 4, 5]], table[[0, 9, 0, 3]])
        np.testing.assert_array_equal(got[[2, 3]], 0.0)


def _splitk_case(rng, kind, m, n, k):
    """A GEMM of the split-K shape family with bias + ReLU + residual: args and host operands."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    a32 = rng.standard_normal((m, k)).astype(np.float32)
    b32 = rng.standard_normal((n, k)).astype(np.float32)
    if kind == "fp32":
        a_st, b_st, code, odt, ocode = a32, b32, _lib.F32, np.float32, _lib.F32
        res_st = rng.standard_normal((m, n)).astype(np.float32)
    else:
        (a_st, _), (b_st, _) = _bits(a32, kind), _bits(b32, kind)
        code = _lib.BF16 if kind == "bf16" else _lib.F16
        odt, ocode = (BF16, _lib.BF16) if kind == "bf16" else (np.float16, _lib.F16)
        res_st, _ = _bits(rng.standard_normal((m, n)).astype(np.float32), kind)
    keep = [_dev(a_st), _dev(b_st), _dev(rng.standard_normal(n).astype(np.float32)), _dev(res_st)]
    ad, bd, biasd, resd = keep
    g = _lib.GemmArgs()
    g.a, g.b, g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = ad.ptr, bd.ptr, m, n, k, k, k, n, 1
    g.trans_a, g.trans_b, g.in_dtype, g.out_dtype = 0, 1, code, ocode
    g.epi = E.epilogue(bias=biasd, bias_mode=2, act=1, residual=resd, alpha=0.75)
    return g, keep, odt


@pytest.mark.parametrize("kind,m,n,k,splits", [("fp32", 256, 512, 784, 16), ("bf16", 256, 1000, 512, 8),
                                               ("fp16", 100, 72, 1024, 4), ("fp32", 3, 7, 40, 5)])
def test_gemm_splitk_one_call_equals_two_launches(gpu, kind, m, n, k, splits):
    """c3h_gemm_splitk (partials in a caller workspace + ordered reduce) is bit
    for bit the compiled engine's two launches (batched partial GEMM, then
    c3h_gemm_splitk_reduce); a workspace one element short is refused."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(m * 7 + n + k)
    g, keep, odt = _splitk_case(rng, kind, m, n, k)
    ws = DeviceArray.empty((splits, m, n), np.float32)
    out1 = DeviceArray.empty((m, n), odt)
    g.out = out1.ptr
    E.gemm_splitk(g, splits, ws)
    # the same two launches by hand
    part = DeviceArray.empty((splits, m, n), np.float32)
    out2 = DeviceArray.empty((m, n), odt)
    p = _lib.GemmArgs()
    C.memmove(C.byref(p), C.byref(g), C.sizeof(g))
    ks = k // splits
    p.out, p.k, p.batch, p.stride_a, p.stride_b, p.stride_out, p.out_dtype = part.ptr, ks, splits, ks, ks, m * n, _lib.F32
    p.epi = E.epilogue()
    _lib.launch(p, None)
    r = _lib.SplitKArgs()
    r.partial, r.out, r.m, r.n, r.ldo, r.splits, r.out_dtype, r.epi = part.ptr, out2.ptr, m, n, n, splits, \
        g.out_dtype, g.epi
    _lib.launch(r, None)
    a, b = out1.get(), out2.get()
    np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8))
    assert np.any(a.view(np.uint8) != 0)
    # a workspace one byte short is refused before any launch
    short = DeviceArray.empty((splits * m * n - 1,), np.float32)
    rc = _lib.lib().c3h_gemm_splitk(C.byref(g), splits, short.ptr, short.nbytes, None)
    assert rc != 0 and "workspace" in _lib.last_error()


@pytest.mark.parametrize("rows,cols,dt,res", [(16 * 1024, 768, "bf16", False), (37, 512, "fp16", True),
                                              (5, 1024, "fp32", True), (9, 24, "bf16", False),
                                              (16 * 1024, 768, "bf16", True)])
def test_layernorm_int8_output_equals_layernorm_then_quantize(gpu, rows, cols, dt, res):
    """LayerNorm with the QuantizeLinear fused (out_dtype I8, the W8A8 pre-LN
    inputs) gives exactly the codes of LayerNorm -> stored activation ->
    c3h_quantize, including saturated codes and a nonzero zero point."""
    from hackathon_amd import _lib
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(rows * 3 + cols)
    x32 = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    r32 = rng.standard_normal((rows, cols)).astype(np.float32)
    if dt == "fp32":
        xd, rd, code, sdt = _dev(x32), _dev(r32), _lib.F32, np.float32
    else:
        xd, rd = _dev(_bits(x32, dt)[0]), _dev(_bits(r32, dt)[0])
        code, sdt = (_lib.BF16, BF16) if dt == "bf16" else (_lib.F16, np.float16)
    gd = _dev(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    bd = _dev(rng.standard_normal(cols).astype(np.float32) * 0.1)
    qscale, qzero = 0.019, -3  # some codes saturate at +-127/-128
    mid = DeviceArray.empty((rows, cols), sdt)
    codes_a = DeviceArray.empty((rows, cols), np.int8)
    codes_b = DeviceArray.empty((rows, cols), np.int8)

    def ln(out, out_code):
        a = _lib.LayerNormArgs()
        a.x, a.residual, a.scale, a.bias, a.out = xd.ptr, rd.ptr if res else None, gd.ptr, bd.ptr, out.ptr
        a.rows, a.cols, a.epsilon, a.x_dtype, a.out_dtype = rows, cols, 1e-5, code, out_code
        a.out_scale, a.out_zero = qscale, qzero
        _lib.launch(a, None)

    print(f"layernorm->int8 rows={rows} cols={cols} {dt} res={res}", flush=True)
    ln(mid, code)
    q = _lib.QuantizeArgs()
    q.x, q.out, q.count, q.scale, q.zero_point, q.x_dtype = mid.ptr, codes_a.ptr, rows * cols, qscale, qzero, code
    _lib.launch(q, None)
    codes_b.copy_from_host(np.full(rows * cols, 77, np.int8))
    ln(codes_b, _lib.I8)
    a_, b_ = codes_a.get(), codes_b.get()
    np.testing.assert_array_equal(a_, b_)
    assert (a_ == 127).any() and (a_ == -128).any()


_with_env = switches.with_switch


@pytest.mark.parametrize("kind", ["bf16", "fp16", "int8"])
@pytest.mark.parametrize("m,n,k", [(300, 200, 64), (256, 128, 128), (130, 70, 192), (1000, 256, 320),
                                   (4096, 512, 1152), (512, 64, 576), (2048, 2048, 512)])
def test_gemm_register_pipelined_matches_two_stage(gpu, kind, m, n, k):
    """The register-pipelined DMA kernel (2, 3 or 4 LDS stages) is bit for bit
    the two-stage kernel: same K order, same accumulation, same epilogue --
    for K tile counts below, at and above the stage count, ragged M/N and a
    bias + residual + ReLU epilogue (int8: requantize -> dequantize mode 3)."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(m + 3 * n + 7 * k)
    bias = _dev(rng.standard_normal(n).astype(np.float32))
    if kind == "int8":
        a = _dev(rng.integers(-128, 128, size=(m, k), dtype=np.int8))
        b = _dev(rng.integers(-127, 128, size=(n, k), dtype=np.int8))
        sb = _dev((rng.random(n) * 0.01 + 0.001).astype(np.float32))
        res = _dev(_bits(rng.standard_normal((m, n)).astype(np.float32), "bf16")[0])
        out = DeviceArray.empty((m, n), BF16)
    else:
        a = _dev(_bits(rng.standard_normal((m, k)).astype(np.float32), kind)[0])
        b = _dev(_bits(rng.standard_normal((n, k)).astype(np.float32), kind)[0])
        res = _dev(_bits(rng.standard_normal((m, n)).astype(np.float32), kind)[0])
        out = DeviceArray.empty((m, n), BF16 if kind == "bf16" else np.float16)

    def run():
        out.copy_from_host(np.zeros(out.nbytes, np.uint8))
        if kind == "int8":
            g = _lib.QGemmArgs()
            g.a, g.b, g.out, g.m, g.n, g.k, g.lda, g.ldb, g.ldo = a.ptr, b.ptr, out.ptr, m, n, k, k, k, n
            g.a_scale, g.y_scale, g.b_scale, g.mode, g.out_dtype = 0.02, 0.37, sb.ptr, 3, _lib.BF16
            g.epi = E.epilogue(bias=bias, bias_mode=2, act=1, residual=res)
        else:
            g = _lib.GemmArgs()
            g.a, g.b, g.out, g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = a.ptr, b.ptr, out.ptr, m, n, k, k, k, n, 1
            code = _lib.BF16 if kind == "bf16" else _lib.F16
            g.trans_a, g.trans_b, g.in_dtype, g.out_dtype = 0, 1, code, code
            g.epi = E.epilogue(bias=bias, bias_mode=2, act=1, residual=res)
        _lib.launch(g, None)
        return out.get().copy()

    print(f"register pipelining {kind} {m}x{n}x{k}", flush=True)
    want = _with_env("C3H_DISABLE_BIGTILE", "1", lambda: _with_env("C3H_DMA_RP", "0", run))
    assert np.any(want.view(np.uint8) != 0)
    for rp in ("2", "3", "4"):
        got = _with_env("C3H_DISABLE_BIGTILE", "1", lambda: _with_env("C3H_DMA_RP", rp, run))
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8), err_msg=f"RP stages {rp}")


@pytest.mark.parametrize("n,hw,c,o,kh,stride", [(256, 28, 128, 128, 3, 1), (256, 56, 64, 128, 3, 2),
                                                (8, 14, 256, 256, 3, 1), (16, 7, 512, 512, 3, 1),
                                                (32, 28, 128, 256, 1, 2)])
def test_conv_register_pipelined_matches_two_stage(gpu, n, hw, c, o, kh, stride):
    """Tap-uniform implicit-GEMM convs (the ResNet-18 layer 2-4 shapes) on the
    register-pipelined kernel are bit-identical to the two-stage kernel."""
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(n + hw + c + o + kh)
    pad = kh // 2
    ho = (hw + 2 * pad - kh) // stride + 1
    x, _ = _bits(rng.standard_normal((n, hw, hw, c)).astype(np.float32), "bf16")
    kpack = ((kh * kh * c + 31) // 32) * 32
    w = np.zeros((o, kpack), np.float32)
    w[:, :kh * kh * c] = rng.standard_normal((o, kh * kh * c)).astype(np.float32) * 0.05
    wb, _ = _bits(w, "bf16")
    res, _ = _bits(rng.standard_normal((n, ho, ho, o)).astype(np.float32), "bf16")
    xd, wd, rd = _dev(x), _dev(wb), _dev(res)
    bd = _dev(rng.standard_normal(o).astype(np.float32))
    out = DeviceArray.empty((n, ho, ho, o), BF16)

    def run():
        out.copy_from_host(np.zeros(out.nbytes, np.uint8))
        a = _lib.ConvArgs()
        a.x, a.w, a.out = xd.ptr, wd.ptr, out.ptr
        a.n, a.c, a.h, a.w_, a.c_stride, a.c_pack, a.o = n, c, hw, hw, c, c, o
        a.kh, a.kw, a.sh, a.sw, a.pad_top, a.pad_left, a.dh, a.dw, a.ho, a.wo = kh, kh, stride, stride, pad, pad, \
            1, 1, ho, ho
        a.out_layout, a.in_dtype, a.out_dtype = 1, _lib.BF16, _lib.BF16
        a.epi = E.epilogue(bias=bd, bias_mode=2, act=1, residual=rd)
        _lib.launch(a, None)
        return out.get().copy()

    print(f"register pipelining conv n={n} {hw}x{hw} c={c} o={o} k={kh} s={stride}", flush=True)
    want = _with_env("C3H_DISABLE_BIGTILE", "1", lambda: _with_env("C3H_DMA_RP", "0", run))
    assert np.any(want.view(np.uint8) != 0)
    for rp in ("2", "3", "4"):
        got = _with_env("C3H_DISABLE_BIGTILE", "1", lambda: _with_env("C3H_DMA_RP", rp, run))
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8), err_msg=f"RP stages {rp}")


@pytest.mark.parametrize("kind", ["fp32", "bf16", "fp16"])
def test_nonfinite_flag(gpu, kind):
    """c3h_nonfinite: the flag is set by any NaN / +-Inf (vector body and the
    ragged tail), never by finite values including the largest and subnormals."""
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    code = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16}[kind]
    big = {"fp32": np.finfo(np.float32).max, "bf16": 3.3895314e38, "fp16": 65504.0}[kind]
    tiny = {"fp32": 1e-45, "bf16": 1e-39, "fp16": 6e-8}[kind]
    rng = np.random.default_rng(3)
    flag = DeviceArray.empty((1,), np.int32)

    def run(x32):
        host = x32.astype(np.float32) if kind == "fp32" else _bits(x32.astype(np.float32), kind)[0]
        xd = _dev(host)
        flag.copy_from_host(np.zeros(1, np.int32))
        a = _lib.NonfiniteArgs()
        a.x, a.flag, a.count, a.dtype = xd.ptr, flag.ptr, x32.size, code
        _lib.launch(a, None)
        return int(flag.get()[0])

    for n in (1, 7, 8, 1000, 4099, 1 << 20):
        x = rng.standard_normal(n).astype(np.float32)
        x[0], x[-1] = big, -big
        if n > 2:
            x[n // 2] = tiny
        print(f"nonfinite {kind} n={n}", flush=True)
        assert run(x) == 0
        for pos in sorted({0, n // 3, n - 1}):
            for bad in (np.nan, np.inf, -np.inf):
                y = x.copy()
                y[pos] = bad
                assert run(y) == 1, (n, pos, bad)
