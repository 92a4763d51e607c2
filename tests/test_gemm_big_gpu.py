"""Bit-exact parity of the large-M GEMM path (256 x 128 tiles, used from 8192
rows: the encoder's QKV / out-projection / FC1+GeLU / FC2+residual15 and the
channels-last conv1/conv2) against the CPU oracle.

Shapes take ragged M and N (partial tiles on both edges), the model's K
values, and the conv geometries of the encoder front end at full length.
"""
import numpy as np
import pytest
import torch

from tests import gen

pytestmark = pytest.mark.gpu

BIG_ROWS = 8192


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("M,K,N", [(BIG_ROWS, 64, 128), (8300, 1280, 200), (9000, 512, 1536),
                                   (BIG_ROWS + 1, 5120, 130), (12345, 768, 77)])
@pytest.mark.parametrize("has_bias,asym", [(True, True), (False, True), (True, False)])
def test_linear8_big(iw, oracle, gpu, M, K, N, has_bias, asym):
    print("case: linear8_big", M, K, N, has_bias, asym, flush=True)
    x, w, b, z, m, s = gen.realistic_linear_case(M + K + N + has_bias, M, K, N, has_bias=has_bias,
                                                 asym=asym)
    s[:3] = [-1, 0, 32][: min(3, N)]  # shift outside [0, 31] gives 0; shift 0 is the identity
    got = iw.kernels.linear8_hip(T(x), T(w), None if b is None else T(b),
                                 None if z is None else T(z), T(m), T(s))
    exp = oracle.linear8(x, w, b, z, m, s)
    assert np.array_equal(host(got), exp)
    assert len(np.unique(exp)) > 100


@pytest.mark.parametrize("M,K,N", [(8300, 1280, 200), (BIG_ROWS + 5, 5120, 64)])
def test_linear32_big(iw, oracle, gpu, M, K, N):
    print("case: linear32_big", M, K, N, flush=True)
    x, w, b, z, m, s = gen.linear_case(M + 7 * N, M, K, N, shift_lo=0, shift_hi=40)
    got = iw.kernels.linear32_hip(T(x), T(w), T(b), T(z), T(m), T(s))
    assert np.array_equal(host(got), oracle.linear32(x, w, b, z, m, s))


@pytest.mark.parametrize("M,K,N,pci,pco", [(8300, 1280, 300, True, True), (8300, 1280, 300, False, False),
                                           (8300, 1280, 300, False, True), (8300, 1280, 300, True, False),
                                           (BIG_ROWS, 384, 1536, True, True), (BIG_ROWS, 384, 1536, False, False)])
def test_linear8_gelu_big(iw, oracle, gpu, M, K, N, pci, pco):
    """Per-channel and per-tensor GeLU parameters (both per-tensor: the GEMM
    applies GeLU as a table of the int8 value)."""
    print("case: linear8_gelu_big", M, K, N, pci, pco, flush=True)
    x, w, b, z, m, s = gen.realistic_linear_case(M + K + 3 * N, M, K, N)
    r = gen.rng(M * N + pci + 2 * pco)
    lut, im, is_, om, os_ = gen.gelu_params(r, N, pci, pco)
    got = iw.kernels.linear8_gelu_hip(T(x), T(w), T(b), T(z), T(m), T(s), T(lut), T(im), T(is_),
                                      T(om), T(os_))
    exp = oracle.gelu(oracle.linear8(x, w, b, z, m, s), lut, im, is_, om, os_)
    assert np.array_equal(host(got), exp)


@pytest.mark.parametrize("ishift,oshift,im,om", [(40, 7, 200, 255), (-3, 33, 1, 128), (0, 0, 255, 255), (13, -1, 0, 77)])
def test_linear8_gelu_big_table_edge_params(iw, oracle, gpu, ishift, oshift, im, om):
    """One GeLU parameter set for all columns (the table form) with shifts
    outside [0, 31] and zero multipliers, which the decoding clamps."""
    M, K, N = 8300, 640, 160
    print("case: linear8_gelu_big table", ishift, oshift, im, om, flush=True)
    x, w, b, z, m, s = gen.realistic_linear_case(M + ishift + 7 * oshift, M, K, N)
    lut = np.sort(gen.rng(5).integers(0, 256, size=16)).astype(np.uint8)
    pi = (np.array([im], np.uint8), np.array([ishift], np.int8))
    po = (np.array([om], np.uint8), np.array([oshift], np.int8))
    got = iw.kernels.linear8_gelu_hip(T(x), T(w), T(b), T(z), T(m), T(s), T(lut), T(pi[0]), T(pi[1]),
                                      T(po[0]), T(po[1]))
    exp = oracle.gelu(oracle.linear8(x, w, b, z, m, s), lut, pi[0], pi[1], po[0], po[1])
    assert np.array_equal(host(got), exp)


@pytest.mark.parametrize("M,K,N", [(8300, 2048, 200), (BIG_ROWS + 100, 5120, 128)])
def test_linear32_residual15_big(iw, oracle, gpu, M, K, N):
    print("case: linear32_residual15_big", M, K, N, flush=True)
    x, w, b, z, m, s = gen.realistic_linear_case(M * 3 + K + N, M, K, N)
    s[:] = np.arange(N) % 3
    r = gen.rng(M + N)
    res = r.integers(-16383, 16384, size=(M, N)).astype(np.int16)
    rm = int(r.integers(1, 65536))
    exp = oracle.residual15(oracle.linear32(x, w, b, z, m, s), res, rm)
    rt = T(res)
    iw.kernels.linear32_residual15_hip(T(x), T(w), T(b), T(z), T(m), T(s), rt,
                                       torch.tensor([rm], dtype=torch.uint16), out=rt)
    assert np.array_equal(host(rt), exp)
    assert len(np.unique(exp)) > 1000


@pytest.mark.parametrize("M,K,N", [(8300, 384, 1000)])
def test_classifier_big(iw, oracle, gpu, M, K, N):
    print("case: classifier_big", M, K, N, flush=True)
    r = gen.rng(M + N)
    x = gen.i8(r, (1, M, K))
    w = gen.i8(r, (N, K))
    for mult, shift in ((int(r.integers(2**28, 2**32)), 10), (0x80000000, -3), (12345, 40)):
        got = iw.kernels.classifier_hip(T(x), T(w), torch.tensor([mult], dtype=torch.uint32),
                                        torch.tensor([shift], dtype=torch.int8))
        assert np.array_equal(host(got), oracle.classifier(x, w, mult, shift))


def _kc(w, cin, ks):
    cout = w.shape[0]
    return np.ascontiguousarray(w.reshape(cout, cin, ks).transpose(0, 2, 1).reshape(cout, ks * cin))


@pytest.mark.parametrize("B,Cin,Tin,Cout,stride", [(3, 80, 3000, 384, 1), (3, 128, 3000, 256, 1),
                                                   (6, 384, 3000, 200, 2), (2, 16, 5000, 32, 1)])
def test_conv1d_channels_last_big(iw, oracle, gpu, B, Cin, Tin, Cout, stride):
    """The encoder front end at full length: conv -> GeLU (-> positional add_requant15)."""
    print("case: conv1d_cl_big", B, Cin, Tin, Cout, stride, flush=True)
    r = gen.rng(B * Cin + Tin + Cout)
    x = gen.i8(r, (B, Cin, Tin))
    w = gen.i8(r, (Cout, Cin * 3), -60, 60)
    bias = r.integers(-2**16, 2**16, size=Cout).astype(np.int32)
    mult, shift = int(r.integers(2**29, 2**31)), 10
    lut, im, is_, om, os_ = gen.gelu_params(r, Cout, False, True)
    conv = oracle.conv1d(x, w, bias, mult, shift, stride, 1)
    assert len(np.unique(conv)) > 60
    g = oracle.gelu(np.ascontiguousarray(conv.transpose(0, 2, 1)), lut, im, is_, om, os_)
    tout = g.shape[1]
    xcl = T(np.ascontiguousarray(x.transpose(0, 2, 1)))
    wkc = T(_kc(w, Cin, 3))
    bt, lt, imt, ist, omt, ost = T(bias), T(lut), T(im), T(is_), T(om), T(os_)
    out8 = torch.empty((B, tout, Cout), dtype=torch.int8, device="cuda")
    iw._lib.call("iw_conv1d_cl", xcl.data_ptr(), wkc.data_ptr(), bt.data_ptr(), mult, shift,
                 lt.data_ptr(), imt.data_ptr(), ist.data_ptr(), omt.data_ptr(), ost.data_ptr(), 1,
                 Cout, None, None, None, 0, 0, out8.data_ptr(), B, Cin, Tin, Cout, 3, stride, 1,
                 True, stream())
    assert np.array_equal(host(out8), g)
    pe = gen.i8(r, (tout, Cout))
    pm = r.integers(1, 65536, size=Cout).astype(np.uint16)
    ps = r.integers(-1, 12, size=Cout).astype(np.int8)
    exp16 = oracle.add_requant15(g, pe, pm, ps)
    out16 = torch.empty((B, tout, Cout), dtype=torch.int16, device="cuda")
    pe_t, pm_t, ps_t = T(pe), T(pm), T(ps)
    iw._lib.call("iw_conv1d_cl", xcl.data_ptr(), wkc.data_ptr(), bt.data_ptr(), mult, shift,
                 lt.data_ptr(), imt.data_ptr(), ist.data_ptr(), omt.data_ptr(), ost.data_ptr(), 1,
                 Cout, pe_t.data_ptr(), pm_t.data_ptr(), ps_t.data_ptr(), Cout, Cout,
                 out16.data_ptr(), B, Cin, Tin, Cout, 3, stride, 1, True, stream())
    assert np.array_equal(host(out16), exp16)


# The direct-to-LDS GEMM (K % 64 == 0, N % 16 == 0) at shapes with several
# times more 256 x 256 tiles than the GPU has CUs, ragged M (and N) edges,
# in-place residual, per-tensor GeLU (the table form) and multipliers on both
# sides of 2^31.
@pytest.mark.parametrize("kind,M,K,N", [("l8", 12000, 1280, 3840), ("l8_sym", 12000, 1280, 3840),
                                        ("l8_bigmult", 12000, 768, 5120), ("gelu_table", 12000, 1280, 5120),
                                        ("l32res", 20000, 1280, 1040), ("l32res_k5120", 9000, 5120, 1280),
                                        ("l32", 17000, 512, 2048)])
def test_gemm_many_tiles(iw, oracle, gpu, kind, M, K, N):
    print("case: gemm many tiles", kind, M, K, N, flush=True)
    seed = M + K + N + len(kind)
    if kind == "l8_bigmult":
        x, w, b, z, m, s = gen.linear_case(seed, M, K, N, shift_lo=0, shift_hi=40)
    else:
        x, w, b, z, m, s = gen.realistic_linear_case(seed, M, K, N, asym=kind != "l8_sym")
    if kind in ("l8", "l8_sym", "l8_bigmult"):
        got = iw.kernels.linear8_hip(T(x), T(w), T(b), None if z is None else T(z), T(m), T(s))
        exp = oracle.linear8(x, w, b, z, m, s)
    elif kind == "gelu_table":
        lut, im, is_, om, os_ = gen.gelu_params(gen.rng(seed), N, False, False)
        got = iw.kernels.linear8_gelu_hip(T(x), T(w), T(b), T(z), T(m), T(s), T(lut), T(im), T(is_), T(om), T(os_))
        exp = oracle.gelu(oracle.linear8(x, w, b, z, m, s), lut, im, is_, om, os_)
    elif kind == "l32":
        got = iw.kernels.linear32_hip(T(x), T(w), T(b), T(z), T(m), T(s))
        exp = oracle.linear32(x, w, b, z, m, s)
    else:
        s[:] = np.arange(N) % 4
        r = gen.rng(seed + 1)
        res = r.integers(-16383, 16384, size=(M, N)).astype(np.int16)
        rm = int(r.integers(1, 65536))
        exp = oracle.residual15(oracle.linear32(x, w, b, z, m, s), res, rm)
        got = T(res)
        iw.kernels.linear32_residual15_hip(T(x), T(w), T(b), T(z), T(m), T(s), got,
                                           torch.tensor([rm], dtype=torch.uint16), out=got)
    assert np.array_equal(host(got), exp)
    assert len(np.unique(exp)) > 100


# Edge shapes of the direct-to-LDS GEMM (K % 64 == 0, N % 16 == 0): a few
# dozen tiles, the narrowest N, partial 256-column blocks, a short K (four
# 64-byte steps) and a long one, with and without zero points and with the
# GeLU table.
@pytest.mark.parametrize("M,K,N", [(8448, 256, 256), (8269, 1280, 16), (9001, 320, 1040), (8200, 5120, 272),
                                   (16384 + 129, 768, 2304)])
@pytest.mark.parametrize("kind", ["asym", "sym", "gelu_table"])
def test_linear8_dtl_edge_shapes(iw, oracle, gpu, M, K, N, kind):
    print("case: linear8 dtl edge", kind, M, K, N, flush=True)
    seed = 3 * M + 5 * K + N + len(kind)
    x, w, b, z, m, s = gen.realistic_linear_case(seed, M, K, N, asym=kind != "sym")
    s[: min(4, N)] = [-2, 0, 33, 31][: min(4, N)]
    if kind == "gelu_table":
        lut, im, is_, om, os_ = gen.gelu_params(gen.rng(seed), N, False, False)
        got = iw.kernels.linear8_gelu_hip(T(x), T(w), T(b), T(z), T(m), T(s), T(lut), T(im), T(is_), T(om), T(os_))
        exp = oracle.gelu(oracle.linear8(x, w, b, z, m, s), lut, im, is_, om, os_)
    else:
        got = iw.kernels.linear8_hip(T(x), T(w), T(b), None if z is None else T(z), T(m), T(s))
        exp = oracle.linear8(x, w, b, z, m, s)
    assert np.array_equal(host(got), exp)
    assert len(np.unique(exp)) > (20 if kind == "gelu_table" else 50)
