"""GPU parity of every registry kernel against the NumPy oracle.

Each case runs the same kernel name through hackathon_amd's HIP registry and
through oracle/registry_ref.py on identical inputs (the reference's own test
fixtures where it has them: linspace/arange ramps from c33/test_fused_kernels.py
and c35/test_c35.py, default_rng(7) from c32/test_kernel_registry.py).
Tolerances: fp32 rtol 1e-5..1e-4 as in those tests; integer/byte/index work
bit-exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import registry_ref as R

pytestmark = pytest.mark.gpu


def _dev(x):
    from hackathon_amd.device import DeviceArray

    return None if x is None else DeviceArray.from_host(np.ascontiguousarray(x))


def run_both(name, inputs, params, n_out=1, capacity=None):
    """Run kernel `name` on the GPU registry and the oracle; return (gpu, ref) lists."""
    from hackathon_amd.c32 import kernel_registry as K
    from hackathon_amd.device import DeviceArray, synchronize

    cap = capacity or [4096] * n_out
    dev_in = [_dev(x) for x in inputs]
    dev_out = [DeviceArray.empty((c,), np.float32) for c in cap]
    K.lookup(name)(dev_in, dev_out, dict(params), None)
    synchronize()
    ref_out = [np.zeros(c, np.float32) for c in cap]
    R.lookup(name)([None if x is None else np.asarray(x) for x in inputs], ref_out, dict(params), None)
    return [o.get() for o in dev_out], ref_out


def check(name, inputs, params, rtol=1e-5, atol=1e-6, n_out=1, capacity=None):
    got, ref = run_both(name, inputs, params, n_out, capacity)
    for g, r in zip(got, ref):
        assert g.shape == r.shape, (g.shape, r.shape)
        np.testing.assert_allclose(g.astype(np.float64), r.astype(np.float64), rtol=rtol, atol=atol)
    return got, ref


def lin(lo, hi, shape, dtype=np.float32):
    return np.linspace(lo, hi, math.prod(shape), dtype=dtype).reshape(shape)


# -- elementwise -------------------------------------------------------------------------------------
def test_elementwise_binary_broadcast(gpu):
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    b = np.array([1.0, -1.0, 2.0, -2.0], np.float32)
    check("add_f32", [x, b], {})
    check("sub_f32", [x, b], {})
    check("mul_f32", [lin(-3, 3, (2, 3, 4)), np.array([0.5, 1.0, 1.5, 2.0], np.float32)], {})
    check("div_f32", [np.arange(1, 13, dtype=np.float32).reshape(3, 4), np.array([1, 2, 4, 8], np.float32)], {})
    check("add_f32", [lin(-1, 1, (5, 1, 7)), lin(2, 3, (1, 6, 1))], {})


def test_elementwise_unary(gpu):
    x = lin(-3, 3, (2, 3, 40))
    check("relu_f32", [x], {})
    check("erf_f32", [x], {}, rtol=1e-6, atol=1e-6)  # A&S 7.1.26 on both sides
    check("exp_f32", [x], {}, rtol=2e-6)
    check("sqrt_f32", [np.abs(x) + 0.1], {})
    check("reciprocal_f32", [np.abs(x) + 0.1], {})
    check("add", [x], {"epsilon": 1e-5})


def test_erf_as_error_bound(gpu):
    """A&S 7.1.26 stays within its published 1.5e-7 of the true erf (float64)."""
    from scipy.special import erf

    x = lin(-4, 4, (4001,))
    got, _ = run_both("erf_f32", [x], {}, capacity=[4001])
    assert np.max(np.abs(got[0].astype(np.float64) - erf(x.astype(np.float64)))) < 1.5e-7 + 2e-7


# -- reductions ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("params", [{"axis": -1, "keepdims": True}, {"axis": 1, "keepdims": True},
                                    {"axes": [-2, -1], "keepdims": True}, {"axis": 0, "keepdims": False}, {}])
def test_reductions(gpu, params):
    x = lin(-2, 5, (3, 5, 7, 9))
    check("reduce_max", [x], params)
    check("reduce_sum", [x], params, rtol=1e-5, atol=1e-4)
    check("reduce_mean_f32", [x], params, rtol=1e-5, atol=1e-5)


# -- matmul / gemm / conv lowering ------------------------------------------------------------------------
@pytest.mark.parametrize("m,n,k", [(1, 1, 2), (3, 4, 2), (37, 19, 23), (128, 96, 64), (200, 300, 260)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul_gemm_lowering(gpu, m, n, k, ta, tb):
    rng = np.random.default_rng(m * 131 + n * 7 + k)
    a = rng.standard_normal((k, m) if ta else (m, k), dtype=np.float32)
    b = rng.standard_normal((n, k) if tb else (k, n), dtype=np.float32)
    check("matmul_f32", [a, b], {"transA": ta, "transB": tb, "alpha": 0.5, "lowering_kind": "gemm"},
          rtol=1e-4, atol=1e-4, capacity=[m * n])


def test_matmul_batched_broadcast(gpu):
    a = np.arange(2 * 1 * 3 * 4, dtype=np.float32).reshape(2, 1, 3, 4)
    b = np.arange(5 * 4 * 2, dtype=np.float32).reshape(1, 5, 4, 2)
    check("matmul_f32", [a, b], {"lowering_kind": "matmul"}, rtol=1e-5, atol=1e-4)
    q = lin(-0.5, 0.5, (2, 3, 5, 7))
    v = lin(0.4, -0.4, (2, 3, 7, 5))
    check("matmul_f32", [q, v], {"lowering_kind": "matmul"}, rtol=1e-5, atol=1e-5)


def test_im2col_contract_reshape_bias_matches_nchw_convolution(gpu):
    """c32/test_kernel_registry.py:52-105 fixture: rectangular kernel, asymmetric pads, stride 2."""
    from hackathon_amd.c32 import kernel_registry as K
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 2, 4, 5), dtype=np.float32)
    weight = rng.standard_normal((3, 2, 3, 2), dtype=np.float32)
    bias = rng.standard_normal((3,), dtype=np.float32)
    params = {"kernel_shape": [3, 2], "strides": [1, 2], "dilations": [1, 1], "pads": [1, 0, 1, 1],
              "lowering_kind": "conv_contract", "_batch_size": 2, "_output_spatial": [4, 3]}
    cols = [DeviceArray.empty((24 * 12,), np.float32)]
    K.lookup("im2col_f32")([_dev(x)], cols, params, None)
    contract = [DeviceArray.empty((24 * 3,), np.float32)]
    K.lookup("matmul_f32")([cols[0], _dev(weight)], contract, params, None)
    shaped = [DeviceArray.empty((72,), np.float32)]
    K.lookup("conv_reshape_f32")([contract[0]], shaped, params, None)
    out = [DeviceArray.empty((72,), np.float32)]
    K.lookup("add_bias_f32")([shaped[0], _dev(bias)], out, {"bias_axis": 1}, None)
    got = out[0].get()
    padded = np.pad(x, ((0, 0), (0, 0), (1, 1), (0, 1)))
    expected = np.empty((2, 3, 4, 3), np.float32)
    for n in range(2):
        for o in range(3):
            for h in range(4):
                for w in range(3):
                    expected[n, o, h, w] = np.sum(padded[n, :, h:h + 3, w * 2:w * 2 + 2] * weight[o]) + bias[o]
    np.testing.assert_allclose(got, expected, rtol=1e-5, atol=1e-5)
    # and the oracle agrees with the brute force too
    ref = R.conv2d(x, weight, params, bias)
    np.testing.assert_allclose(ref, expected, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("case", [
    dict(x=(2, 4, 7, 7), w=(6, 4, 3, 3), pads=[1, 1, 1, 1], strides=[1, 1], dil=[1, 1]),
    dict(x=(1, 3, 32, 32), w=(16, 3, 3, 3), pads=[0, 0, 0, 0], strides=[2, 2], dil=[1, 1]),
    dict(x=(2, 5, 11, 9), w=(7, 5, 3, 2), pads=[1, 0, 2, 1], strides=[1, 2], dil=[2, 1]),
    dict(x=(2, 64, 9, 9), w=(128, 64, 1, 1), pads=[0, 0, 0, 0], strides=[2, 2], dil=[1, 1]),
    dict(x=(1, 3, 23, 23), w=(16, 3, 7, 7), pads=[3, 3, 3, 3], strides=[2, 2], dil=[1, 1]),
])
def test_winograd_step_is_a_convolution(gpu, case):
    rng = np.random.default_rng(11)
    x = rng.standard_normal(case["x"], dtype=np.float32)
    w = rng.standard_normal(case["w"], dtype=np.float32)
    params = {"kernel_shape": list(case["w"][2:]), "pads": case["pads"], "strides": case["strides"],
              "dilations": case["dil"], "group": 1}
    check("winograd_forward_f32", [x, w], params, rtol=1e-4, atol=1e-4, capacity=[100000])


def test_conv_same_lower_dilation_and_group(gpu):
    """c35/test_c35.py:402-426 closed forms."""
    from hackathon_amd.c35 import engine as E

    x = np.arange(30, dtype=np.float32).reshape(1, 1, 5, 6)
    w = np.array([[[[1.0, 2.0], [3.0, 4.0]]]], np.float32)
    got = E.op_conv([_dev(x), _dev(w)], {"auto_pad": "SAME_LOWER", "strides": [2, 2], "dilations": [2, 2],
                                         "group": 1}).get()
    p = np.pad(x, ((0, 0), (0, 0), (1, 1), (1, 0)))
    exp = p[:, :, 0:6:2, 0:6:2] * 1 + p[:, :, 0:6:2, 2:8:2] * 2 + p[:, :, 2:8:2, 0:6:2] * 3 + p[:, :, 2:8:2, 2:8:2] * 4
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-6)
    gx = np.arange(18, dtype=np.float32).reshape(1, 2, 3, 3)
    gw = np.array([[[[2.0]]], [[[3.0]]]], np.float32)
    got = E.op_conv([_dev(gx), _dev(gw)], {"group": 2}).get()
    np.testing.assert_array_equal(got[:, 0], gx[:, 0] * 2.0)
    np.testing.assert_array_equal(got[:, 1], gx[:, 1] * 3.0)


def test_batchnorm(gpu):
    x = lin(-1, 1, (2, 3, 4, 5))
    s, b, m, v = lin(0.5, 1.5, (3,)), lin(-0.2, 0.2, (3,)), lin(-0.1, 0.1, (3,)), lin(0.1, 1.6, (3,))
    check("batchnorm_f32", [x, s, b, m, v], {"epsilon": 1e-5}, rtol=1e-5, atol=1e-5)


# -- fused ops (c33/test_fused_kernels.py:36-175 fixtures) ---------------------------------------------
def test_fused_softmax_nonlast_axis(gpu):
    check("fused_softmax_f32", [lin(-3, 3, (2, 5, 7))], {"axis": 1}, rtol=1e-5, atol=1e-6)
    check("fused_softmax_f32", [lin(-2, 2, (3, 11))], {"axis": -1}, rtol=1e-5, atol=1e-6)
    check("fused_softmax_f32", [lin(-30, 30, (4, 3000))], {"axis": -1}, rtol=1e-5, atol=1e-7,
          capacity=[12000])


def test_fused_residual_norm(gpu):
    x = lin(-1, 1, (3, 4, 16))
    r = lin(0.5, -0.5, (3, 4, 16))
    check("fused_residual_norm_f32", [x, r, lin(0.75, 1.25, (16,)), lin(-0.1, 0.1, (16,))],
          {"axis": -1, "epsilon": 1e-5}, rtol=1e-4, atol=1e-5)


def test_fused_layer_norm_wide_and_narrow(gpu):
    check("fused_layer_norm_f32", [lin(-2, 2, (3, 5, 16)), lin(0.8, 1.2, (16,)), lin(-0.1, 0.1, (16,))],
          {"axis": -1, "epsilon": 1e-5}, rtol=1e-4, atol=1e-5)
    check("fused_layer_norm_f32", [lin(-2, 2, (3, 3000)), lin(0.8, 1.2, (3000,))],
          {"axis": -1, "epsilon": 1e-5}, rtol=1e-4, atol=1e-5, capacity=[9000])


def test_layer_norm_axis_one_three_outputs(gpu):
    """c35/test_c35.py:453-471."""
    from hackathon_amd.c35 import engine as E

    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    scale, bias = lin(0.5, 1.5, (3, 4)), lin(-0.2, 0.2, (3, 4))
    y, mean, inv = E.op_layer_normalization([_dev(x), _dev(scale), _dev(bias)],
                                            {"axis": 1, "epsilon": 1e-3, "_num_outputs": 3})
    em = x.mean(axis=(1, 2), keepdims=True)
    c = x - em
    ei = 1.0 / np.sqrt((c * c).mean(axis=(1, 2), keepdims=True) + 1e-3)
    np.testing.assert_allclose(y.get(), c * ei * scale + bias, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(mean.get(), em, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(inv.get(), ei, rtol=1e-6, atol=1e-6)


def test_fused_gemm_flatten_bias_relu(gpu):
    x = lin(-1, 1, (2, 3, 4))
    w = lin(-0.5, 0.5, (12, 5))
    b = lin(-0.2, 0.2, (5,))
    got, _ = check("fused_gemm_epilogue_f32", [x, w, b], {"_flatten_axis": 1, "_activation": "Relu"},
                   rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(got[0], np.maximum(x.reshape(2, 12) @ w + b, 0), rtol=1e-5, atol=1e-5)


def test_fused_gemm_transposes_alpha_beta_bias_modes(gpu):
    """c35/test_c35.py:386-397 plus every C broadcast mode of E:771-793."""
    a = np.arange(6, dtype=np.float32).reshape(3, 2)
    b = np.arange(12, dtype=np.float32).reshape(3, 4)
    for c in (np.linspace(-1, 1, 4, dtype=np.float32), np.float32(0.5) * np.ones((1, 1), np.float32),
              lin(-1, 1, (2, 1)), lin(-1, 1, (2, 4))):
        got, _ = check("fused_gemm_epilogue_f32", [a, b, c], {"transA": 1, "alpha": 0.5, "beta": 2.0},
                       rtol=1e-6, atol=1e-5)
        np.testing.assert_allclose(got[0], 0.5 * (a.T @ b) + 2.0 * c, rtol=1e-6, atol=1e-5)


def test_fused_matmul_bias_batched(gpu):
    x = lin(-1, 1, (2, 3, 7))
    w = lin(-0.4, 0.4, (7, 5))
    b = lin(-0.1, 0.1, (5,))
    got, _ = check("fused_matmul_bias_f32", [x, w, b], {}, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(got[0], np.matmul(x, w) + b, rtol=1e-5, atol=1e-5)


def test_fused_ew_chain_programs(gpu):
    x = np.array([[-2.0, 1.0]], np.float32)
    c1 = np.array([[3.0, 4.0]], np.float32)
    c2 = np.array([[10.0, 20.0]], np.float32)
    ops = [{"op": "Add", "attrs": {}, "inputs": [0, 1], "output": "t0"},
           {"op": "Mul", "attrs": {}, "inputs": ["t0", 2], "output": "t1"},
           {"op": "Relu", "attrs": {}, "inputs": ["t1"], "output": "y"}]
    got, _ = check("fused_ew_f32", [x, c1, c2], {"_ops": ops})
    np.testing.assert_allclose(got[0], np.maximum((x + c1) * c2, 0), rtol=1e-6, atol=1e-6)
    # GELU chain (Div -> Erf -> Add -> Mul -> Mul) on a [rows, cols] tensor with scalar constants
    f = lin(-4, 4, (6, 50))
    gelu = [{"op": "Div", "inputs": [0, 1], "output": "a"}, {"op": "Erf", "inputs": ["a"], "output": "b"},
            {"op": "Add", "inputs": ["b", 2], "output": "c"}, {"op": "Mul", "inputs": [0, "c"], "output": "d"},
            {"op": "Mul", "inputs": ["d", 3], "output": "e"}]
    consts = [np.array([math.sqrt(2.0)], np.float32), np.array([1.0], np.float32), np.array([0.5], np.float32)]
    check("fused_ew_f32", [f] + consts, {"_ops": gelu}, rtol=2e-6, atol=2e-6)


def test_fused_attention_scores(gpu):
    q = lin(-0.5, 0.5, (2, 3, 5, 7))
    kt = lin(0.4, -0.4, (2, 3, 7, 5))
    div = np.asarray([7.0 ** 0.5], np.float32)
    mask = lin(-0.2, 0.2, (1, 1, 5, 5))
    check("fused_attention_scores_f32", [q, kt, div, mask], {"axis": -1}, rtol=1e-4, atol=1e-5)
    # broadcast batch/head and a causal -inf mask
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 4, 9, 8), dtype=np.float32)
    kt = rng.standard_normal((2, 1, 8, 9), dtype=np.float32)
    m = np.triu(np.full((9, 9), -np.inf, np.float32), 1)
    check("fused_attention_scores_f32", [q, kt, np.asarray([8.0 ** 0.5], np.float32), m], {"axis": -1},
          rtol=1e-4, atol=1e-6)


def test_fused_transpose_reshape(gpu):
    v = np.arange(120, dtype=np.float32).reshape(2, 3, 4, 5)
    got, _ = check("fused_transpose_reshape_f32", [v, np.array([2, 4, 15], np.int64)],
                   {"perm": [0, 2, 1, 3], "allowzero": 0}, rtol=0, atol=0)
    np.testing.assert_array_equal(got[0], v.transpose(0, 2, 1, 3).reshape(2, 4, 15))


def test_fused_residual_relu(gpu):
    check("fused_residual_relu_f32", [lin(-1, 1, (2, 6, 7, 7)), lin(0.2, -0.2, (2, 6, 7, 7))], {})


# -- data movement -------------------------------------------------------------------------------
def test_reshape_transpose_flatten_split_gather(gpu):
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    check("reshape", [x, np.array([0, -1], np.int64)], {"allowzero": 0}, rtol=0, atol=0)
    check("transpose", [x], {"perm": None}, rtol=0, atol=0)
    check("transpose", [lin(0, 1, (1, 4, 18, 32))], {"perm": [0, 2, 1, 3]}, rtol=0, atol=0)
    check("flatten", [np.arange(120, dtype=np.float32).reshape(2, 3, 4, 5)], {"axis": 2}, rtol=0, atol=0)
    check("split", [np.arange(24, dtype=np.float32).reshape(2, 12)], {"axis": -1, "split": [2, 4, 6],
                                                                       "_num_outputs": 3}, n_out=3, rtol=0, atol=0)
    check("split", [lin(0, 1, (1, 18, 384))], {"axis": -1, "split": [], "_num_outputs": 3}, n_out=3,
          rtol=0, atol=0, capacity=[8000] * 3)
    data = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    check("gather", [data, np.array([[3, 1], [0, 2]], np.int64)], {"axis": -1}, rtol=0, atol=0)
    emb = lin(-1, 1, (50, 64))
    check("gather", [emb, np.array([[0, 49, 7], [-1, 3, 3]], np.int64)], {"axis": 0}, rtol=0, atol=0)


def test_gather_preserves_int64_in_engine(gpu):
    from hackathon_amd.c35 import engine as E

    data = np.arange(24, dtype=np.int64).reshape(2, 3, 4)
    idx = np.array([[3, 1], [0, 2]], np.int64)
    got = E.op_gather([_dev(data), _dev(idx)], {"axis": -1})
    assert got.dtype == np.int64
    np.testing.assert_array_equal(got.get(), np.take(data, idx, axis=2))


# -- rows the reference lacks ---------------------------------------------------------------------
def test_maxpool(gpu):
    x = np.random.default_rng(5).standard_normal((2, 3, 13, 13)).astype(np.float32)
    check("maxpool_f32", [x], {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]}, rtol=0, atol=0)
    check("maxpool_f32", [x], {"kernel_shape": [2, 3], "strides": [1, 2], "pads": [0, 1, 1, 0],
                               "dilations": [2, 1]}, rtol=0, atol=0)


def test_quantize_qlinear_matmul_dequantize_bit_exact(gpu):
    from hackathon_amd.c32 import kernel_registry as K
    from hackathon_amd.device import DeviceArray, synchronize

    rng = np.random.default_rng(9)
    x = rng.standard_normal((48, 64), dtype=np.float32) * 3
    x[0, :4] = [0.5, 1.5, 2.5, -0.5]  # exact halves: round half to even
    sa = np.array(0.5 / 1.0, np.float32)
    for fn_name, ins in [("quantize_linear", [x, sa, np.array(0, np.int8)])]:
        got = [DeviceArray.empty((48 * 64,), np.float32)]
        K.lookup(fn_name)([_dev(v) for v in ins], got, {}, None)
        synchronize()
        q = got[0].get().view(np.int8)[:48 * 64].reshape(48, 64)
        np.testing.assert_array_equal(q, R.quantize(x, sa, 0))
    assert list(q[0, :4]) == [1, 3, 5, -1]
    wq = rng.integers(-127, 128, size=(64, 40), dtype=np.int8)
    sw = (rng.random(40) * 0.01 + 0.001).astype(np.float32)
    sy = np.array(0.75, np.float32)
    z8 = np.array(0, np.int8)
    ins = [q, sa, z8, wq, sw, np.zeros(40, np.int8), sy, z8]
    out = [DeviceArray.empty((48 * 40,), np.float32)]
    K.lookup("qlinear_matmul")([_dev(v) for v in ins], out, {}, None)
    synchronize()
    got_q = out[0].get().view(np.int8)[:48 * 40].reshape(48, 40)
    np.testing.assert_array_equal(got_q, R.requantize(R.qlinear_matmul_acc(q, 0, wq, 0), sa, sw, sy, 0))
    check("dequantize_linear", [got_q, sy, z8], {}, rtol=0, atol=0)


def test_qgemm_int32_accumulators_bit_exact(gpu):
    """int8 MFMA accumulators equal exact integer products (mode 0) at MI355X tile edges."""
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(21)
    for m, n, k in [(1, 1, 16), (130, 70, 3072), (257, 129, 96)]:
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        bt = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        out = DeviceArray.empty((m, n), np.int32)
        E.qgemm(_dev(a), _dev(bt), out, m, n, k, mode=0)
        np.testing.assert_array_equal(out.get(), (a.astype(np.int64) @ bt.T.astype(np.int64)).astype(np.int32))
    a = np.full((4, 3072), -128, np.int8)
    bt = np.full((4, 3072), -127, np.int8)  # extreme: 3072 * 128 * 127
    out = DeviceArray.empty((4, 4), np.int32)
    E.qgemm(_dev(a), _dev(bt), out, 4, 4, 3072, mode=0)
    assert int(out.get()[0, 0]) == 3072 * 128 * 127


def _argmax_both(x, params, rows):
    from hackathon_amd.c32 import kernel_registry as K
    from hackathon_amd.device import DeviceArray, synchronize

    out = [DeviceArray.empty((2 * rows,), np.float32)]
    K.lookup("argmax")([_dev(x)], out, dict(params), None)
    synchronize()
    ref = [np.zeros(rows, np.int64)]
    R.lookup("argmax")([x], ref, dict(params), None)
    return out[0].get().view(np.int64).reshape(-1)[:rows], ref[0].reshape(-1)


def test_argmax_ties_and_nan(gpu):
    x = np.array([[1, 3, 3, 2], [0, 0, 0, 0], [-1, np.nan, 5, np.nan], [2, 1, 0, -1]], np.float32)
    got, ref = _argmax_both(x, {"axis": -1, "keepdims": 0}, 4)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got, [1, 0, 1, 0])  # first max; NaN wins like NumPy
    big = np.random.default_rng(2).standard_normal((33, 32000)).astype(np.float32)
    got, ref = _argmax_both(big, {"axis": -1, "keepdims": 1}, 33)
    np.testing.assert_array_equal(got, ref)


def test_unknown_kernel_fails_closed(gpu):
    from hackathon_amd.c32 import kernel_registry as K

    with pytest.raises(RuntimeError, match="Unknown kernel"):
        K.lookup("sigmoid_f32")
