"""Fragment-major decode operands: the packing kernel against a numpy
restatement of the layout, and every *_frag entry point bit-exact against the
oracle on the same seeded inputs (fragment-major results are unpacked by the
numpy restatement before the comparison)."""
import numpy as np
import pytest
import torch

from tests import gen

pytestmark = pytest.mark.gpu


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def stream():
    return torch.cuda.current_stream().cuda_stream


def kpad(k):
    return (k + 319) // 320 * 320


def rpad(r):
    return (r + 31) // 32 * 32


def frag_image(x):
    """[R, K] int8 -> its fragment-major bytes: blocks of 32 rows x 32 k, each
    64 lanes x 16 bytes, lane l = row % 32 + 32 * (k // 16 % 2)."""
    R, K = x.shape
    p = np.zeros((rpad(R), kpad(K)), np.int8)
    p[:R, :K] = x
    return p.reshape(rpad(R) // 32, 32, kpad(K) // 32, 2, 16).transpose(0, 2, 3, 1, 4).reshape(-1)


def unfrag(buf, R, K):
    b = np.asarray(buf).reshape(rpad(R) // 32, kpad(K) // 32, 2, 32, 16).transpose(0, 3, 1, 2, 4)
    return b.reshape(rpad(R), kpad(K))[:R, :K]


def pack(iw, x):
    R, K = x.shape
    out = torch.full((iw._lib.value("iw_frag_bytes", R, K),), 77, dtype=torch.int8, device="cuda")
    xt = T(x)
    iw._lib.call("iw_frag_pack", xt.data_ptr(), R, K, K, out.data_ptr(), stream())
    torch.cuda.synchronize()
    return out


def zeros_frag(iw, R, K):
    return torch.zeros(iw._lib.value("iw_frag_bytes", R, K), dtype=torch.int8, device="cuda")


@pytest.mark.parametrize("R,K", [(1, 1), (70, 700), (128, 1280), (33, 5120), (51865, 64)])
def test_frag_pack(iw, R, K):
    print("case: frag pack", R, K, flush=True)
    x = gen.i8(gen.rng(R + K), (R, K))
    got = host(pack(iw, x))
    assert np.array_equal(got, frag_image(x))
    assert np.array_equal(unfrag(got, R, K), x)


FRAG_SHAPES = [(1, 1280, 1280), (128, 1280, 1280), (128, 1280, 3840), (128, 1280, 5120),
               (128, 5120, 1280), (37, 384, 1536), (5, 1536, 384), (100, 2048, 200),
               (128, 4096, 64), (77, 640, 96)]


@pytest.mark.parametrize("M,K,N", FRAG_SHAPES)
@pytest.mark.parametrize("has_bias,asym", [(True, True), (False, False)])
def test_linear8_frag(iw, oracle, gpu, M, K, N, has_bias, asym):
    print("case: linear8_frag", M, K, N, has_bias, asym, flush=True)
    x, w, b, z, m, s = gen.linear_case(M * 5 + K + N, M, K, N, has_bias=has_bias, asym=asym,
                                       shift_lo=-2, shift_hi=34)
    exp = oracle.linear8(x, w, b, z, m, s)
    xf, wf = pack(iw, x), pack(iw, w)
    bt, zt, mt, st = (None if b is None else T(b)), (None if z is None else T(z)), T(m), T(s)
    ptr = lambda t: None if t is None else t.data_ptr()
    out = torch.empty((M, N), dtype=torch.int8, device="cuda")
    args = (xf.data_ptr(), wf.data_ptr(), ptr(bt), ptr(zt), mt.data_ptr(), st.data_ptr())
    iw._lib.call("iw_linear8_frag", *args, out.data_ptr(), M, K, N, has_bias, asym, False, stream())
    torch.cuda.synchronize()
    assert np.array_equal(host(out), exp)
    if N <= 5120:
        of = zeros_frag(iw, M, N)
        iw._lib.call("iw_linear8_frag", *args, of.data_ptr(), M, K, N, has_bias, asym, True, stream())
        torch.cuda.synchronize()
        got = host(of)
        assert np.array_equal(unfrag(got, M, N), exp)
        # nothing is written into the padding
        assert np.array_equal(got, frag_image(exp))


@pytest.mark.parametrize("M,K,N", [(128, 1280, 5120), (7, 384, 1536), (100, 1280, 300)])
def test_linear8_gelu_frag(iw, oracle, gpu, M, K, N):
    print("case: linear8_gelu_frag", M, K, N, flush=True)
    x, w, b, z, m, s = gen.realistic_linear_case(M + K + N, M, K, N)
    lut, im, is_, om, os_ = gen.gelu_params(gen.rng(M * N), N, True, True)
    exp = oracle.gelu(oracle.linear8(x, w, b, z, m, s), lut, im, is_, om, os_)
    xf, wf = pack(iw, x), pack(iw, w)
    ts = [T(a) for a in (b, z, m, s, lut, im, is_, om, os_)]
    # without and with the prefetch hint (the next GEMM's weight, N2 x K2):
    # the same output
    r = gen.rng(M + 2 * N)
    n2, k2 = (1280, 5120) if K == 1280 else (33, 700)
    nxt = pack(iw, gen.i8(r, (n2, k2)))
    for pf in ((None, 0, 0), (nxt.data_ptr(), n2, k2)):
        of = zeros_frag(iw, M, N)
        iw._lib.call("iw_linear8_gelu_frag", xf.data_ptr(), wf.data_ptr(), *[t.data_ptr() for t in ts], N, N,
                     of.data_ptr(), M, K, N, True, True, True, *pf, stream())
        torch.cuda.synchronize()
        assert np.array_equal(host(of), frag_image(exp)), pf[1:]


@pytest.mark.parametrize("M,K,N", [(128, 1280, 1280), (128, 5120, 1280), (37, 1536, 384), (1, 2560, 64),
                                   (100, 4096, 1024)])
def test_linear32_residual15_frag(iw, oracle, gpu, M, K, N):
    print("case: linear32_residual15_frag", M, K, N, flush=True)
    x, w, b, z, m, s = gen.realistic_linear_case(M * 3 + K + N, M, K, N)
    r = gen.rng(M + N)
    res = r.integers(-16383, 16384, size=(M, N)).astype(np.int16)
    rm = int(r.integers(1, 65536))
    exp = oracle.residual15(oracle.linear32(x, w, b, z, m, s), res, rm)
    xf, wf = pack(iw, x), pack(iw, w)
    ts = [T(a) for a in (b, z, m, s)]
    rt = T(res)  # in place on the residual stream, as the decoder uses it
    iw._lib.call("iw_linear32_residual15_frag", xf.data_ptr(), wf.data_ptr(), *[t.data_ptr() for t in ts],
                 rt.data_ptr(), rm, rt.data_ptr(), M, K, N, True, True, stream())
    torch.cuda.synchronize()
    assert np.array_equal(host(rt), exp)


@pytest.mark.parametrize("M,K,N", [(128, 1280, 51865), (1, 384, 51865), (3, 512, 1000), (64, 512, 20000),
                                   (97, 768, 17000)])
def test_classifier_frag(iw, oracle, gpu, M, K, N):
    print("case: classifier_frag", M, K, N, flush=True)
    r = gen.rng(M + K + N)
    x = gen.i8(r, (M, K))
    w = gen.i8(r, (N, K))
    xf, wf = pack(iw, x), pack(iw, w)
    for mult, shift in ((int(r.integers(2**28, 2**32)), 10), (0x80000000, -3), (12345, 40)):
        out = torch.empty((M, N), dtype=torch.int8, device="cuda")
        iw._lib.call("iw_classifier_frag", xf.data_ptr(), wf.data_ptr(), mult, shift, out.data_ptr(), M, K, N,
                     stream())
        torch.cuda.synchronize()
        assert np.array_equal(host(out), oracle.classifier(x[None], w, mult, shift)[0])


@pytest.mark.parametrize("hidden,rows", [(384, 1), (1280, 128), (512, 37), (1024, 100)])
def test_layernorm32_frag(iw, oracle, gpu, hidden, rows):
    print("case: layernorm32_frag", hidden, rows, flush=True)
    x, g, b, lm, ls, om, os_ = gen.ln_case(hidden * 3 + rows, rows, hidden, 4000)
    exp = oracle.layernorm32(x, g, b, lm, ls, om, os_)
    xt, gt, bt = T(x), T(g), T(b)
    # without and with the prefetch hint (a QKV-shaped next weight, and one
    # with fewer column tiles than XCDs): the same output
    nxt = pack(iw, gen.i8(gen.rng(rows + hidden), (3 * hidden, hidden)))
    for pf in ((None, 0, 0), (nxt.data_ptr(), 3 * hidden, hidden), (nxt.data_ptr(), 70, hidden)):
        of = zeros_frag(iw, rows, hidden)
        iw._lib.call("iw_layernorm32_frag", xt.data_ptr(), gt.data_ptr(), bt.data_ptr(), lm, ls, om, os_, 13,
                     of.data_ptr(), rows, hidden, True, *pf, stream())
        torch.cuda.synchronize()
        assert np.array_equal(host(of), frag_image(exp)), pf[1:]


def test_layernorm32_frag_rejects_many_rows(iw, gpu):
    x = torch.zeros((129, 384), dtype=torch.int16, device="cuda")
    g = torch.zeros(384, dtype=torch.int8, device="cuda")
    of = zeros_frag(iw, 129, 384)
    with pytest.raises(RuntimeError, match="at most 128 rows"):
        iw._lib.call("iw_layernorm32_frag", x.data_ptr(), g.data_ptr(), None, 1, 1, 1, 1, 13, of.data_ptr(),
                     129, 384, False, None, 0, 0, stream())


def test_frag_prefetch_hint_is_checked(iw, gpu):
    x = torch.zeros((4, 384), dtype=torch.int16, device="cuda")
    g = torch.zeros(384, dtype=torch.int8, device="cuda")
    of = zeros_frag(iw, 4, 384)
    w = zeros_frag(iw, 64, 384)
    for n, k, what in ((64, 6000, "prefetch weight shape"), (0, 384, "prefetch weight shape"),
                       (64, 384, "16-byte aligned")):
        ptr = w.data_ptr() + (4 if what == "16-byte aligned" else 0)
        with pytest.raises(RuntimeError, match=what):
            iw._lib.call("iw_layernorm32_frag", x.data_ptr(), g.data_ptr(), None, 1, 1, 1, 1, 13,
                         of.data_ptr(), 4, 384, False, ptr, n, k, stream())


@pytest.mark.parametrize("B,H,D,Tk,tcap,k_length,layout", [
    (2, 3, 64, 17, 448, 1, "vt"), (128, 20, 64, 1500, 1500, 1500, "vt"), (3, 4, 96, 100, 448, 1, "vt"),
    (1, 2, 128, 300, 448, 1, "vt"), (2, 3, 64, 17, 448, 1, "quads"), (128, 20, 64, 301, 448, 1, "quads"),
    (5, 20, 64, 448, 448, 1, "quads_pad")])
def test_attention_decode_cache_frag(iw, oracle, gpu, B, H, D, Tk, tcap, k_length, layout):
    print("case: decode cache frag", B, H, D, Tk, tcap, k_length, layout, flush=True)
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(5 * B + Tk + D, B, H, 1, Tk, D)
    exp = oracle.attention(q, k, v, None, qm, qs, f, am, as_).reshape(B, H * D)
    kc = np.zeros((B, H, tcap, D), np.int8)
    shape, vs = gen.v_cache_layout(B, H, D, tcap, layout)
    vc = np.zeros(shape, np.int8)
    kc[:, :, :Tk] = k
    gen.v_cache_put(vc, layout, 0, v)  # attn_case gives V transposed, [B, H, D, Tk]
    qt, kt, vt = T(q.reshape(B, H * D)), T(kc), T(vc)
    pos_val = None if k_length == Tk else Tk - k_length
    pos = None if pos_val is None else torch.tensor([pos_val], dtype=torch.int32, device="cuda")
    max_keys = tcap if pos is not None else k_length
    of = zeros_frag(iw, B, H * D)
    iw._lib.call("iw_attention_decode_cache_frag", qt.data_ptr(), H * D, kt.data_ptr(), H * tcap * D, tcap * D,
                 D, vt.data_ptr(), *vs, of.data_ptr(), B, H, D, k_length,
                 None if pos is None else pos.data_ptr(), max_keys, qm, qs, f, am, as_, 16, None, 0, 0,
                 stream())
    torch.cuda.synchronize()
    assert np.array_equal(host(of), frag_image(exp))


@pytest.mark.parametrize("B,H,Tk,next_n,next_k", [(2, 3, 17, 64, 192), (128, 20, 301, 1280, 1280),
                                                  (128, 20, 448, 1280, 1280), (7, 4, 5, 96, 256)])
def test_attention_decode_cache_frag_prefetch_hint(iw, oracle, gpu, B, H, Tk, next_n, next_k):
    """The self-attention kernel's last blocks read a next-GEMM weight into L2:
    a hint that changes no result (grids smaller and larger than the tail,
    weights of fewer column tiles than XCDs and of many)."""
    print("case: decode cache frag prefetch", B, H, Tk, next_n, next_k, flush=True)
    D, tcap = 64, 448
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(11 * B + Tk, B, H, 1, Tk, D)
    exp = oracle.attention(q, k, v, None, qm, qs, f, am, as_).reshape(B, H * D)
    kc = np.zeros((B, H, tcap, D), np.int8)
    shape, vs = gen.v_cache_layout(B, H, D, tcap, "quads")
    vc = np.zeros(shape, np.int8)
    kc[:, :, :Tk] = k
    gen.v_cache_put(vc, "quads", 0, v)
    qt, kt, vt = T(q.reshape(B, H * D)), T(kc), T(vc)
    wn = pack(iw, gen.i8(gen.rng(B + Tk), (next_n, next_k)))
    for hint in ((None, 0, 0), (wn.data_ptr(), next_n, next_k)):
        of = zeros_frag(iw, B, H * D)
        iw._lib.call("iw_attention_decode_cache_frag", qt.data_ptr(), H * D, kt.data_ptr(), H * tcap * D,
                     tcap * D, D, vt.data_ptr(), *vs, of.data_ptr(), B, H, D, Tk, None, Tk, qm, qs, f, am, as_,
                     16, *hint, stream())
        torch.cuda.synchronize()
        assert np.array_equal(host(of), frag_image(exp))


@pytest.mark.parametrize("B,H,D,pos_val,tcap", [(128, 20, 64, 100, 448), (5, 6, 64, 447, 448),
                                                (3, 4, 96, 0, 448), (2, 2, 64, 40, 40)])
@pytest.mark.parametrize("layout", gen.V_LAYOUTS)
def test_linear8_qkv_cache_frag(iw, oracle, gpu, B, H, D, pos_val, tcap, layout):
    print("case: qkv cache frag", B, H, D, pos_val, tcap, layout, flush=True)
    C = H * D
    x, w, b, z, m, s = gen.realistic_linear_case(B + C + pos_val, B, C, 3 * C)
    exp = oracle.linear8(x, w, b, z, m, s)
    r = gen.rng(9)
    kc0 = gen.i8(r, (B, H, tcap, D))
    shape, vs = gen.v_cache_layout(B, H, D, tcap, layout)
    vc0 = gen.i8(r, shape)
    kc, vc = T(kc0), T(vc0)
    q = torch.empty((B, C), dtype=torch.int8, device="cuda")
    pos = torch.tensor([pos_val], dtype=torch.int32, device="cuda")
    xf, wf = pack(iw, x), pack(iw, w)
    ts = [T(a) for a in (b, z, m, s)]
    iw._lib.call("iw_linear8_qkv_cache_frag", xf.data_ptr(), wf.data_ptr(), *[t.data_ptr() for t in ts], B, C,
                 True, True, q.data_ptr(), C, kc.data_ptr(), H * tcap * D, tcap * D, D, vc.data_ptr(),
                 *vs, C, D, 1, tcap, pos.data_ptr(), stream())
    torch.cuda.synchronize()
    assert np.array_equal(host(q), exp[:, :C])
    kexp, vexp = kc0.copy(), vc0.copy()
    e = exp.reshape(B, 3, H, D)
    if pos_val < tcap:
        kexp[:, :, pos_val, :] = e[:, 1]
        gen.v_cache_put(vexp, layout, pos_val, e[:, 2][..., None])
    assert np.array_equal(host(kc), kexp)
    assert np.array_equal(host(vc), vexp)


def test_frag_gemm_rejects_large_k(iw, gpu):
    x = torch.zeros(iw._lib.value("iw_frag_bytes", 4, 5120), dtype=torch.int8, device="cuda")
    m = torch.ones(8, dtype=torch.int32, device="cuda")
    s = torch.zeros(8, dtype=torch.int8, device="cuda")
    out = torch.empty((4, 8), dtype=torch.int8, device="cuda")
    with pytest.raises(RuntimeError, match="K <= 5120"):
        iw._lib.call("iw_linear8_frag", x.data_ptr(), x.data_ptr(), None, None, m.data_ptr(), s.data_ptr(),
                     out.data_ptr(), 4, 5440, 8, False, False, False, stream())
