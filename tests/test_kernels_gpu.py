"""Bit-exact parity of every HIP entry point against the CPU oracle.

Each test builds seeded int8/int16/int32 inputs, runs the op on the GPU through
the C ABI (i_whisper_amd.kernels) and on the oracle, and requires equality.
Shapes follow the reference's own test grids (SIMD-width boundaries of K,
head_dim, decode Tq=1 and encoder Tq=Tk geometries) plus the model shapes.
"""
import numpy as np
import pytest
import torch

from tests import gen

pytestmark = pytest.mark.gpu


def T(a, dev="cuda"):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    return t.cpu().numpy()


def _print_case(*args):
    print("case:", *args, flush=True)


# ---------------------------------------------------------------------------
# GEMM family
# ---------------------------------------------------------------------------

GEMM_SHAPES = [
    (1, 1, 1), (3, 15, 5), (7, 16, 9), (5, 17, 33), (33, 31, 64), (64, 32, 128),
    (65, 33, 129), (128, 64, 128), (129, 100, 130), (200, 128, 96), (256, 1280, 384),
    (300, 512, 1536), (1, 1280, 1280), (128, 1280, 1280),
    # decode shapes split over K across blocks (ragged M, few column tiles)
    (100, 2048, 200), (32, 4096, 64), (128, 5120, 1280), (64, 1280, 3840),
]


@pytest.mark.parametrize("M,K,N", GEMM_SHAPES)
@pytest.mark.parametrize("has_bias,asym", [(True, True), (False, True), (True, False), (False, False)])
def test_linear8(iw, oracle, gpu, M, K, N, has_bias, asym):
    _print_case("linear8", M, K, N, has_bias, asym)
    x, w, b, z, m, s = gen.linear_case(M * 7 + K * 13 + N, M, K, N, has_bias=has_bias, asym=asym,
                                       shift_lo=-2, shift_hi=34)
    got = iw.kernels.linear8_hip(T(x), T(w), None if b is None else T(b), None if z is None else T(z),
                                 T(m), T(s))
    exp = oracle.linear8(x, w, b, z, m, s)
    assert np.array_equal(host(got), exp)


@pytest.mark.parametrize("M,K,N", GEMM_SHAPES)
def test_linear8_realistic(iw, oracle, gpu, M, K, N):
    x, w, b, z, m, s = gen.realistic_linear_case(M + 3 * K + 5 * N, M, K, N)
    got = iw.kernels.linear8_hip(T(x), T(w), T(b), T(z), T(m), T(s))
    exp = oracle.linear8(x, w, b, z, m, s)
    assert np.array_equal(host(got), exp)
    if M * N >= 1024:
        assert len(np.unique(exp)) > 16  # not a saturated case


@pytest.mark.parametrize("M,K,N", GEMM_SHAPES)
@pytest.mark.parametrize("has_bias,asym", [(True, True), (False, False)])
def test_linear32(iw, oracle, gpu, M, K, N, has_bias, asym):
    _print_case("linear32", M, K, N)
    x, w, b, z, m, s = gen.linear_case(M * 11 + K + N * 3, M, K, N, has_bias=has_bias, asym=asym,
                                       shift_lo=0, shift_hi=40)
    got = iw.kernels.linear32_hip(T(x), T(w), None if b is None else T(b),
                                  None if z is None else T(z), T(m), T(s))
    exp = oracle.linear32(x, w, b, z, m, s)
    assert np.array_equal(host(got), exp)


@pytest.mark.parametrize("M,K,N", [(5, 17, 33), (128, 64, 128), (300, 512, 1536), (129, 1280, 5120)])
@pytest.mark.parametrize("pc", [True, False])
def test_linear8_gelu(iw, oracle, gpu, M, K, N, pc):
    _print_case("linear8_gelu", M, K, N, pc)
    x, w, b, z, m, s = gen.realistic_linear_case(M + K + N, M, K, N)
    r = gen.rng(M * N)
    lut, im, is_, om, os_ = gen.gelu_params(r, N, pc, pc)
    got = iw.kernels.linear8_gelu_hip(T(x), T(w), T(b), T(z), T(m), T(s), T(lut), T(im), T(is_),
                                      T(om), T(os_))
    exp = oracle.gelu(oracle.linear8(x, w, b, z, m, s), lut, im, is_, om, os_)
    assert np.array_equal(host(got), exp)


@pytest.mark.parametrize("M,K,N", [(5, 17, 33), (128, 64, 128), (300, 2048, 512), (129, 5120, 1280),
                                   (128, 5120, 1280), (77, 1280, 1280)])
def test_linear32_residual15(iw, oracle, gpu, M, K, N):
    _print_case("linear32_residual15", M, K, N)
    x, w, b, z, m, s = gen.realistic_linear_case(M * 3 + K + N, M, K, N)
    r = gen.rng(M + N)
    res = r.integers(-16383, 16384, size=(M, N)).astype(np.int16)
    rm = int(r.integers(1, 65536))
    got = iw.kernels.linear32_residual15_hip(T(x), T(w), T(b), T(z), T(m), T(s), T(res),
                                             torch.tensor([rm], dtype=torch.uint16))
    exp = oracle.residual15(oracle.linear32(x, w, b, z, m, s), res, rm)
    assert np.array_equal(host(got), exp)
    # in place on the residual stream
    rt = T(res)
    iw.kernels.linear32_residual15_hip(T(x), T(w), T(b), T(z), T(m), T(s), rt,
                                       torch.tensor([rm], dtype=torch.uint16), out=rt)
    assert np.array_equal(host(rt), exp)


@pytest.mark.parametrize("M,K,N", [(1, 384, 51865), (3, 384, 1000), (128, 1280, 4099), (2, 17, 33)])
def test_classifier(iw, oracle, gpu, M, K, N):
    _print_case("classifier", M, K, N)
    r = gen.rng(M + K + N)
    x = gen.i8(r, (1, M, K))
    w = gen.i8(r, (N, K))
    for mult, shift in ((int(r.integers(2**28, 2**32)), 10), (0x80000000, -3), (12345, 40)):
        got = iw.kernels.classifier_hip(T(x), T(w), torch.tensor([mult], dtype=torch.uint32),
                                        torch.tensor([shift], dtype=torch.int8))
        exp = oracle.classifier(x, w, mult, shift)
        assert np.array_equal(host(got), exp)


@pytest.mark.parametrize("B,Cin,Tin,Cout,ks,stride,pad", [
    (1, 3, 10, 4, 3, 1, 1), (2, 5, 17, 7, 3, 2, 1), (1, 80, 300, 384, 3, 1, 1),
    (2, 384, 300, 384, 3, 2, 1), (1, 4, 9, 3, 5, 2, 0), (1, 16, 40, 32, 3, 1, 2),
])
def test_conv1d(iw, oracle, gpu, B, Cin, Tin, Cout, ks, stride, pad):
    _print_case("conv1d", B, Cin, Tin, Cout, ks, stride, pad)
    r = gen.rng(B + Cin + Tin + Cout)
    x = gen.i8(r, (B, Cin, Tin))
    w = gen.i8(r, (Cout, Cin * ks))
    bias = r.integers(-2**20, 2**20, size=Cout).astype(np.int32)
    mult, shift = int(r.integers(2**28, 2**32)), 6
    got = iw.kernels.conv1d_hip(T(x), T(w), T(bias), torch.tensor([mult], dtype=torch.uint32),
                                torch.tensor([shift], dtype=torch.int8), stride, pad)
    exp = oracle.conv1d(x, w, bias, mult, shift, stride, pad)
    assert np.array_equal(host(got), exp)


def _kc(w, cin, ks):
    cout = w.shape[0]
    return np.ascontiguousarray(w.reshape(cout, cin, ks).transpose(0, 2, 1).reshape(cout, ks * cin))


@pytest.mark.parametrize("B,Cin,Tin,Cout,stride", [(1, 80, 200, 384, 1), (2, 384, 200, 384, 2),
                                                   (1, 128, 64, 1280, 1), (3, 16, 9, 32, 2)])
def test_conv1d_channels_last_fused(iw, oracle, gpu, B, Cin, Tin, Cout, stride):
    """conv -> gelu (per-tensor in, per-channel out) -> optional positional add_requant15."""
    _print_case("conv1d_cl", B, Cin, Tin, Cout, stride)
    r = gen.rng(B * Cin + Tin)
    x = gen.i8(r, (B, Cin, Tin))
    w = gen.i8(r, (Cout, Cin * 3))
    bias = r.integers(-2**16, 2**16, size=Cout).astype(np.int32)
    mult, shift = int(r.integers(2**29, 2**31)), 8
    lut, im, is_, om, os_ = gen.gelu_params(r, Cout, False, True)
    conv = oracle.conv1d(x, w, bias, mult, shift, stride, 1)  # [B,Cout,Tout]
    g = oracle.gelu(np.ascontiguousarray(conv.transpose(0, 2, 1)), lut, im, is_, om, os_)
    tout = g.shape[1]
    xcl = T(np.ascontiguousarray(x.transpose(0, 2, 1)))
    wkc = T(_kc(w, Cin, 3))
    args = [T(bias), mult, shift, T(lut), T(im), T(is_), T(om), T(os_), 1, Cout]
    out8 = torch.empty((B, tout, Cout), dtype=torch.int8, device="cuda")
    iw._lib.call("iw_conv1d_cl", xcl.data_ptr(), wkc.data_ptr(), args[0].data_ptr(), mult, shift,
                 args[3].data_ptr(), args[4].data_ptr(), args[5].data_ptr(), args[6].data_ptr(),
                 args[7].data_ptr(), 1, Cout, None, None, None, 0, 0, out8.data_ptr(), B, Cin, Tin,
                 Cout, 3, stride, 1, True, torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(host(out8), g)
    pe = gen.i8(r, (tout, Cout))
    pm = r.integers(1, 65536, size=Cout).astype(np.uint16)
    ps = r.integers(-1, 12, size=Cout).astype(np.int8)
    exp16 = oracle.add_requant15(g, pe, pm, ps)
    out16 = torch.empty((B, tout, Cout), dtype=torch.int16, device="cuda")
    pe_t, pm_t, ps_t = T(pe), T(pm), T(ps)
    iw._lib.call("iw_conv1d_cl", xcl.data_ptr(), wkc.data_ptr(), args[0].data_ptr(), mult, shift,
                 args[3].data_ptr(), args[4].data_ptr(), args[5].data_ptr(), args[6].data_ptr(),
                 args[7].data_ptr(), 1, Cout, pe_t.data_ptr(), pm_t.data_ptr(), ps_t.data_ptr(),
                 Cout, Cout, out16.data_ptr(), B, Cin, Tin, Cout, 3, stride, 1, True,
                 torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(host(out16), exp16)


# ---------------------------------------------------------------------------
# Row / element ops
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("hidden", [384, 512, 768, 1024, 1280])
@pytest.mark.parametrize("rows,spread", [(1, 4000), (37, 16000), (1000, 300), (5, 0)])
def test_layernorm32(iw, oracle, gpu, hidden, rows, spread):
    _print_case("layernorm32", hidden, rows, spread)
    x, g, b, lm, ls, om, os_ = gen.ln_case(hidden + rows, rows, hidden, spread)
    got = iw.kernels.layernorm32_hip(
        T(x), T(g), T(b), torch.tensor([lm], dtype=torch.uint8), torch.tensor([ls], dtype=torch.int8),
        torch.tensor([om], dtype=torch.uint32), torch.tensor([os_], dtype=torch.int8))
    exp = oracle.layernorm32(x, g, b, lm, ls, om, os_)
    assert np.array_equal(host(got), exp)


@pytest.mark.parametrize("hidden", [384, 1280])
@pytest.mark.parametrize("rows", [6, 200, 2100])
def test_layernorm32_full_int16_range(iw, oracle, gpu, hidden, rows):
    """Rows whose deviations from the mean exceed 46340, where d^2 wraps in int32
    (the kernels' per-element form), next to ordinary rows in the same launch:
    row-per-block launches (<= 2048 rows) and one persistent-wave launch."""
    _print_case("layernorm32 full int16 range", hidden, rows)
    x, g, b, lm, ls, om, os_ = gen.ln_case(hidden + rows + 1, rows, hidden, 3000)
    r = gen.rng(rows)
    x[0] = 32767
    x[0, 5] = -32768                                     # one deviation of ~65000
    x[1] = np.where(np.arange(hidden) % 2 == 0, -32768, 32767)  # |d| ~ 32767, no wrap
    x[2] = r.integers(-32768, 32768, size=hidden)        # the full range
    x[3] = -32768
    x[3, -1] = 32767
    x[rows // 2] = 30000
    x[rows // 2, ::7] = -30000
    got = iw.kernels.layernorm32_hip(
        T(x), T(g), T(b), torch.tensor([lm], dtype=torch.uint8), torch.tensor([ls], dtype=torch.int8),
        torch.tensor([om], dtype=torch.uint32), torch.tensor([os_], dtype=torch.int8))
    assert np.array_equal(host(got), oracle.layernorm32(x, g, b, lm, ls, om, os_))


@pytest.mark.parametrize("rows", [3, 5000])
def test_layernorm32_unaligned_params(iw, oracle, gpu, rows):
    """gamma / beta views at odd offsets, and no beta at all."""
    hidden = 1280
    _print_case("layernorm32 unaligned", rows)
    x, g, b, lm, ls, om, os_ = gen.ln_case(rows + 7, rows, hidden, 3000)
    gbuf = torch.zeros(hidden + 1, dtype=torch.int8, device="cuda")
    gbuf[1:] = T(g)
    bbuf = torch.zeros(hidden + 1, dtype=torch.int32, device="cuda")
    bbuf[1:] = T(b)
    scal = (torch.tensor([lm], dtype=torch.uint8), torch.tensor([ls], dtype=torch.int8),
            torch.tensor([om], dtype=torch.uint32), torch.tensor([os_], dtype=torch.int8))
    xt = T(x)
    got = iw.kernels.layernorm32_hip(xt, gbuf[1:], bbuf[1:], *scal)
    assert np.array_equal(host(got), oracle.layernorm32(x, g, b, lm, ls, om, os_))
    got = iw.kernels.layernorm32_hip(xt, gbuf[1:], None, *scal)
    assert np.array_equal(host(got), oracle.layernorm32(x, g, None, lm, ls, om, os_))


def test_layernorm32_rejects_width(iw, gpu):
    x = torch.zeros((2, 100), dtype=torch.int16, device="cuda")
    with pytest.raises(RuntimeError, match="unsupported LayerNorm hidden size"):
        iw.kernels.layernorm32_hip(x, torch.zeros(100, dtype=torch.int8, device="cuda"), None,
                                   torch.ones(1, dtype=torch.uint8), torch.zeros(1, dtype=torch.int8),
                                   torch.ones(1, dtype=torch.uint32), torch.zeros(1, dtype=torch.int8))


def test_rsqrt(iw, oracle, gpu):
    vals = {0}
    for bit in range(31):
        for d in (-1, 0, 1):
            v = (1 << bit) + d
            if 0 <= v <= 2**31 - 1:
                vals.add(v)
    r = gen.rng(5)
    x = np.concatenate([np.array(sorted(vals), np.int32),
                        r.integers(0, 1_000_000_001, 4000).astype(np.int32),
                        r.integers(-2**31, 0, 100).astype(np.int32)])
    for off in (13, 16, 0, 29):
        got = iw.kernels.layernorm32_rsqrt_hip(T(x), off)
        assert np.array_equal(host(got), oracle.rsqrt(x, off))


@pytest.mark.parametrize("shape", [(7,), (3, 100), (2, 1500, 384), (4, 33, 1536)])
@pytest.mark.parametrize("pc", [(True, True), (False, True), (False, False)])
def test_gelu(iw, oracle, gpu, shape, pc):
    r = gen.rng(sum(shape))
    x = gen.i8(r, shape)
    lut, im, is_, om, os_ = gen.gelu_params(r, shape[-1], *pc)
    got = iw.kernels.gelu_hip(T(x), T(lut), T(im), T(is_), T(om), T(os_))
    assert np.array_equal(host(got), oracle.gelu(x, lut, im, is_, om, os_))


def test_residual15(iw, oracle, gpu):
    r = gen.rng(3)
    br = r.integers(-2**31, 2**31, size=(3, 77, 384), dtype=np.int64).astype(np.int32)
    res = r.integers(-32768, 32768, size=br.shape).astype(np.int16)
    for m in (0, 1, 32767, 65535):
        got = iw.kernels.residual15_hip(T(br), T(res), torch.tensor([m], dtype=torch.uint16))
        assert np.array_equal(host(got), oracle.residual15(br, res, m))


@pytest.mark.parametrize("pc", [(True, True), (False, False), (True, False)])
def test_add_requant15(iw, oracle, gpu, pc):
    r = gen.rng(11)
    B, Tn, Ch = 2, 50, 384
    x = gen.i8(r, (B, Tn, Ch))
    a = gen.i8(r, (Tn, Ch))
    m = r.integers(0, 65536, size=Ch if pc[0] else 1).astype(np.uint16)
    s = r.integers(-2, 34, size=Ch if pc[1] else 1).astype(np.int8)
    got = iw.kernels.add_requant15_hip(T(x), T(a), T(m), T(s))
    assert np.array_equal(host(got), oracle.add_requant15(x, a, m, s))


# ---------------------------------------------------------------------------
# Attention: op-level kernels and the fused kernels
# ---------------------------------------------------------------------------

ATTN_SHAPES = [(1, 1, 1, 1, 1), (2, 3, 5, 7, 16), (1, 2, 1, 33, 64), (2, 2, 3, 3, 64),
               (1, 4, 64, 64, 64), (1, 2, 130, 150, 96), (1, 1, 1, 1500, 64), (2, 2, 37, 29, 17)]


@pytest.mark.parametrize("B,H,Tq,Tk,D", ATTN_SHAPES)
@pytest.mark.parametrize("masked", [False, True])
def test_attention_ops(iw, oracle, gpu, B, H, Tq, Tk, D, masked):
    _print_case("attention ops", B, H, Tq, Tk, D, masked)
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(B * H + Tq * Tk + D, B, H, Tq, Tk, D)
    mask = gen.causal_mask(Tq, Tk) if masked and Tk >= Tq else None
    qk, rm = iw.kernels.qk_requant_rowmax_hip(T(q), T(k), None if mask is None else T(mask),
                                              torch.tensor([qm], dtype=torch.uint8),
                                              torch.tensor([qs], dtype=torch.int8))
    eqk, erm = oracle.qk_requant_rowmax(q, k, mask, qm, qs)
    assert np.array_equal(host(qk), eqk) and np.array_equal(host(rm), erm)
    p, rs = iw.kernels.shift_exp_hip(qk, rm, None if mask is None else T(mask),
                                     torch.tensor(f, dtype=torch.int32))
    ep, ers = oracle.shift_exp(eqk, erm, mask, f)
    assert np.array_equal(host(p), ep) and np.array_equal(host(rs), ers)
    out = iw.kernels.pv_norm_requant_hip(p, T(v), rs, torch.tensor([am], dtype=torch.uint8),
                                         torch.tensor([as_], dtype=torch.int8), 16)
    assert np.array_equal(host(out), oracle.pv_norm_requant(ep, v, ers, am, as_, 16))


def test_pv_norm_requant_rejects_negative_row_sum(iw, gpu):
    p = torch.zeros((1, 1, 1, 4), dtype=torch.uint8, device="cuda")
    v = torch.zeros((1, 1, 2, 4), dtype=torch.int8, device="cuda")
    rs = torch.tensor([[[[-1]]]], dtype=torch.int32, device="cuda")
    with pytest.raises((RuntimeError, ValueError)):
        iw.kernels.pv_norm_requant_hip(p, v, rs, torch.ones(1, dtype=torch.uint8),
                                       torch.zeros(1, dtype=torch.int8), 16)


def test_shift_exp_wrap_corner(iw, oracle, gpu):
    """Row max 32767 wraps rmp1 to -32768 (attention_scalar.cpp:449-509)."""
    qk = np.array([[[[32767, -32768, 0, 100, -5]]]], np.int16)
    rm = np.array([[[[-32768]]]], np.int16)
    for f in (1, 7, 8, 13):
        p, rs = iw.kernels.shift_exp_hip(T(qk), T(rm), None, torch.tensor(f, dtype=torch.int32))
        ep, ers = oracle.shift_exp(qk, rm, None, f)
        assert np.array_equal(host(p), ep) and np.array_equal(host(rs), ers)


def _fused(iw, q, k, v, mask, qm, qs, f, am, as_, decode):
    """Run the fused kernel on [B,T,H*D] q/k and padded V^T [B,H,D,Tpad]."""
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    qt = T(np.ascontiguousarray(q.transpose(0, 2, 1, 3).reshape(B, Tq, H * D)))
    pad = (Tk + 15) // 16 * 16
    vt = np.zeros((B, H, D, pad), np.int8)
    vt[..., :Tk] = v
    vtt = T(vt)
    out = torch.empty((B, Tq, H * D), dtype=torch.int8, device="cuda")
    if decode:  # K head-major [B,H,Tk,D]
        kt = T(k)
        kstr = (H * Tk * D, Tk * D, D)
    else:       # K as [B,Tk,H*D]
        kt = T(np.ascontiguousarray(k.transpose(0, 2, 1, 3).reshape(B, Tk, H * D)))
        kstr = (Tk * H * D, D, H * D)
    table = None if decode else iw.kernels.shift_exp_table_hip(f)
    iw.kernels.attention_hip(
        qt, kt, vtt, out, batch=B, heads=H, q_length=Tq, k_length=Tk, head_dim=D,
        q_strides=(Tq * H * D, H * D), k_strides=kstr, v_strides=(H * D * pad, D * pad, pad),
        o_strides=(Tq * H * D, H * D), mask=None if mask is None else T(mask), qk_multiplier=qm,
        qk_shift=qs, frac_bits=f, av_multiplier=am, av_shift=as_, rsqrt_offset=16, table=table,
        decode=decode)
    return host(out)


@pytest.mark.parametrize("B,H,Tq,Tk,D", [(1, 1, 1, 1, 64), (1, 2, 5, 7, 64), (2, 3, 130, 150, 64),
                                         (1, 2, 200, 1500, 64), (1, 2, 64, 64, 96), (2, 1, 33, 77, 128),
                                         (1, 1, 40, 40, 16), (1, 2, 300, 300, 32)])
@pytest.mark.parametrize("masked", [False, True])
def test_attention_prefill_fused(iw, oracle, gpu, B, H, Tq, Tk, D, masked):
    _print_case("attention prefill", B, H, Tq, Tk, D, masked)
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(7 * B + Tq + Tk + D, B, H, Tq, Tk, D)
    mask = gen.causal_mask(Tq, Tk) if masked and Tk >= Tq else None
    exp = oracle.attention(q, k, v, mask, qm, qs, f, am, as_)
    got = _fused(iw, q, k, v, mask, qm, qs, f, am, as_, decode=False)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("B,H,Tq,Tk,D", [(1, 1, 1, 1, 64), (2, 3, 1, 1500, 64), (2, 2, 3, 3, 64),
                                         (1, 2, 1, 448, 96), (3, 4, 1, 17, 64), (1, 1, 2, 100, 128),
                                         # several query rows sharing the K/V stream (2, 4 and 8 at
                                         # once), up to the 2048 keys of that path and past them
                                         (2, 20, 3, 1500, 64), (3, 4, 4, 1500, 64), (2, 3, 5, 1500, 64),
                                         (1, 2, 8, 2048, 64), (1, 2, 3, 2100, 64), (2, 2, 7, 129, 64)])
@pytest.mark.parametrize("masked", [False, True])
def test_attention_decode_fused(iw, oracle, gpu, B, H, Tq, Tk, D, masked):
    _print_case("attention decode", B, H, Tq, Tk, D, masked)
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(5 * B + Tq + Tk + D, B, H, Tq, Tk, D)
    mask = gen.causal_mask(Tq, Tk) if masked and Tk >= Tq else None
    exp = oracle.attention(q, k, v, mask, qm, qs, f, am, as_)
    got = _fused(iw, q, k, v, mask, qm, qs, f, am, as_, decode=True)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("decode", [False, True])
def test_attention_fused_wrap_corner(iw, oracle, gpu, decode):
    """Scores saturating at +32767 wrap rmp1 and give P = 128 at x_sub = 0."""
    B, H, Tq, Tk, D = 1, 1, 2, 40, 64
    q = np.full((B, H, Tq, D), 127, np.int8)
    k = np.full((B, H, Tk, D), 127, np.int8)
    k[..., 1::3, :] = -128
    v = gen.i8(gen.rng(1), (B, H, D, Tk))
    exp = oracle.attention(q, k, v, None, 255, 0, 8, 200, 6)
    got = _fused(iw, q, k, v, None, 255, 0, 8, 200, 6, decode)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("qs", [0, 1, 9, 13, 14, 20, 27, 28, 29, 30, 31])
def test_attention_prefill_requant_extremes(iw, oracle, gpu, D, qs):
    """Scores at the int8 extremes (|QK^T| up to 128 * 128 * D) against every
    requant shift and the multipliers 0, 1 and 255, over key chunks that are
    full (64 keys) and a ragged last one: keys aligned with the query (largest
    scores, saturating the int16 row maximum for small shifts), anti-aligned
    (most negative) and random signs."""
    B, H, Tq, Tk = 1, 2, 70, 150
    r = gen.rng(1000 + 31 * D + qs)
    q = np.where(r.random((B, H, Tq, D)) < 0.5, -128, 127).astype(np.int8)
    k = np.where(r.random((B, H, Tk, D)) < 0.5, -128, 127).astype(np.int8)
    for t in range(0, Tk, 5):
        k[:, :, t] = q[:, :, t % Tq]           # aligned with query t % Tq
    for t in range(2, Tk, 7):
        k[:, :, t] = np.where(q[:, :, (t + 3) % Tq] < 0, 127, -128)  # anti-aligned
    v = gen.i8(r, (B, H, D, Tk))
    for qm in (0, 1, 255):
        _print_case("attention prefill extremes", B, H, Tq, Tk, D, f"qs={qs} qm={qm}")
        exp = oracle.attention(q, k, v, None, qm, qs, 8, 200, 6)
        got = _fused(iw, q, k, v, None, qm, qs, 8, 200, 6, decode=False)
        assert np.array_equal(got, exp), (qs, qm)


def test_attention_prefill_wrap_in_full_chunks(iw, oracle, gpu):
    """The row-maximum wrap (P = 128 at x_sub = 0) inside full 64-key chunks:
    every query row saturates at +32767 while a third of the keys sit at
    -32768."""
    B, H, Tq, Tk, D = 1, 2, 33, 200, 64
    q = np.full((B, H, Tq, D), 127, np.int8)
    k = np.full((B, H, Tk, D), 127, np.int8)
    k[..., 1::3, :] = -128
    q[:, 1, 5:] = gen.i8(gen.rng(3), (B, Tq - 5, D))  # rows of head 1 past 5: no saturation
    v = gen.i8(gen.rng(2), (B, H, D, Tk))
    for qs in (0, 4):
        exp = oracle.attention(q, k, v, None, 255, qs, 8, 200, 6)
        got = _fused(iw, q, k, v, None, 255, qs, 8, 200, 6, decode=False)
        assert np.array_equal(got, exp), qs


def test_argmax_rows(iw, gpu):
    r = gen.rng(9)
    x = gen.i8(r, (7, 51865))
    x[3, :] = 5
    x[4, 100] = 127
    x[4, 200] = 127
    got = host(iw.kernels.argmax_rows_hip(T(x)))
    assert np.array_equal(got, np.argmax(x, axis=1))


@pytest.mark.parametrize("cols", [1, 15, 16, 17, 40, 4099, 51865])
def test_argmax_rows_ties_and_alignment(iw, gpu, cols):
    """Rows starting at every offset mod 16 (odd row stride), maxima tied in the
    unaligned head, the 16-byte pieces and the tail, and all-equal rows."""
    r = gen.rng(cols)
    rows = 19
    x = gen.i8(r, (rows, cols))
    x[0, :] = -128
    x[1, :] = 7
    for i in range(2, rows):
        picks = r.integers(0, cols, size=min(3, cols))
        x[i, picks] = 127
    xt = T(x)  # row stride = cols: odd strides put row starts at every alignment
    out = torch.empty(rows, dtype=torch.int64, device="cuda")
    iw._lib.call("iw_argmax_rows", xt.data_ptr(), rows, cols, cols, out.data_ptr(),
                 torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(host(out), np.argmax(x, axis=1))
