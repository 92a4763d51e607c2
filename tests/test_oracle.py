"""Pins the CPU oracle (oracle/iw_oracle.c).

1. Differential: against the reference's own scalar kernels, compiled from the
   reference tree into oracle/_ref (skipped where that build is absent), on
   seeded random inputs over the reference tests' shape grids and on the
   boundary values its tests use.
2. Golden fixtures (tests/golden/*.npz) written from oracle/_ref by
   tests/golden/make_golden.py, so the pin also holds on machines without the
   reference tree.
3. Known answers and closed forms independent of both implementations:
   hand-computed GEMM results from the reference tests, exact int64 matmuls,
   round-half-away-from-zero division, the FISR against 2^off/sqrt(x), and
   brute force over every int8 input for the element-wise ops.
"""
import math

import numpy as np
import pytest

from tests import gen


# ---------------------------------------------------------------------------
# 1. differential against the reference scalar kernels
# ---------------------------------------------------------------------------

LIN_SHAPES = [(1, 1, 1), (2, 3, 2), (3, 15, 5), (4, 16, 4), (5, 17, 7), (7, 31, 9), (8, 32, 8),
              (9, 33, 3), (33, 64, 17), (16, 384, 24)]


@pytest.mark.parametrize("M,K,N", LIN_SHAPES)
@pytest.mark.parametrize("has_bias,asym", [(True, True), (False, True), (True, False), (False, False)])
def test_linear8_vs_ref(oracle, ref, M, K, N, has_bias, asym):
    x, w, b, z, m, s = gen.linear_case(M + K * 3 + N * 7, M, K, N, has_bias=has_bias, asym=asym,
                                       shift_lo=-3, shift_hi=40)
    assert np.array_equal(oracle.linear8(x, w, b, z, m, s), ref.linear8(x, w, b, z, m, s))
    assert np.array_equal(oracle.linear_accum(x, w, b, z), ref.linear_accum(x, w, b, z))


@pytest.mark.parametrize("M,K,N", LIN_SHAPES)
def test_linear32_vs_ref(oracle, ref, M, K, N):
    # shifts in [0, 63]: outside that range the reference C++ shifts by a
    # negative or >= 64 count, which is undefined behaviour
    x, w, b, z, m, s = gen.linear_case(M * 5 + K + N, M, K, N, shift_lo=0, shift_hi=63)
    assert np.array_equal(oracle.linear32(x, w, b, z, m, s), ref.linear32(x, w, b, z, m, s))


@pytest.mark.parametrize("hidden", [384, 512, 768, 1024, 1280])
@pytest.mark.parametrize("spread", [0, 50, 4000, 16383])
def test_layernorm32_vs_ref(oracle, ref, hidden, spread):
    x, g, b, lm, ls, om, os_ = gen.ln_case(hidden + spread, 33, hidden, spread)
    for params in ((lm, ls, om, os_), (255, -20, 0xFFFFFFFF, -1), (1, 0, 1, 40)):
        assert np.array_equal(oracle.layernorm32(x, g, b, *params), ref.layernorm32(x, g, b, *params))
        assert np.array_equal(oracle.layernorm32(x, g, None, *params),
                              ref.layernorm32(x, g, None, *params))


def test_layernorm32_rejects_width(oracle, ref):
    x = np.zeros((2, 100), np.int16)
    g = np.ones(100, np.int8)
    with pytest.raises(ValueError):
        oracle.layernorm32(x, g, None, 1, 0, 1, 0)
    with pytest.raises(ValueError):
        ref.layernorm32(x, g, None, 1, 0, 1, 0)


def test_rsqrt_vs_ref(oracle, ref):
    r = gen.rng(1)
    x = np.concatenate([np.arange(0, 5000, dtype=np.int32),
                        r.integers(-2**31, 2**31, 20000, dtype=np.int64).astype(np.int32),
                        np.array([2**31 - 1, -2**31, 2**30, 2**30 - 1], np.int32)])
    for off in (0, 1, 12, 13, 15, 16, 29):
        assert np.array_equal(oracle.rsqrt(x, off), ref.rsqrt(x, off))


def test_gelu_vs_ref(oracle, ref):
    r = gen.rng(2)
    x = np.arange(-128, 128, dtype=np.int8).repeat(9).reshape(-1, 36)
    for pc in ((True, True), (False, True), (True, False), (False, False)):
        lut, im, is_, om, os_ = gen.gelu_params(r, 36, *pc)
        is_ = is_.copy()
        is_[0] = -5
        if is_.size > 1:
            is_[1] = 40
        assert np.array_equal(oracle.gelu(x, lut, im, is_, om, os_), ref.gelu(x, lut, im, is_, om, os_))


def test_residual15_vs_ref(oracle, ref):
    r = gen.rng(3)
    br = r.integers(-2**31, 2**31, size=5000, dtype=np.int64).astype(np.int32)
    res = r.integers(-32768, 32768, size=5000).astype(np.int16)
    br[:4] = [2**31 - 1, -2**31, 16383 << 15, -(16384 << 15)]
    for m in (0, 1, 2, 32768, 65535):
        assert np.array_equal(oracle.residual15(br, res, m), ref.residual15(br, res, m))


def test_add_requant15_vs_ref(oracle, ref):
    r = gen.rng(4)
    x = gen.i8(r, (2, 9, 24))
    a = gen.i8(r, (9, 24))
    for mc, sc in ((1, 1), (24, 24), (1, 24), (24, 1)):
        m = r.integers(0, 65536, size=mc).astype(np.uint16)
        s = r.integers(-4, 40, size=sc).astype(np.int8)
        assert np.array_equal(oracle.add_requant15(x, a, m, s), ref.add_requant15(x, a, m, s))


@pytest.mark.parametrize("B,Cin,Tin,Cout,ks,stride,pad", [
    (1, 1, 1, 1, 1, 1, 0), (2, 3, 10, 4, 3, 1, 1), (1, 5, 17, 6, 3, 2, 1), (1, 4, 9, 3, 5, 2, 2),
    (2, 8, 31, 5, 3, 3, 0)])
def test_conv1d_vs_ref(oracle, ref, B, Cin, Tin, Cout, ks, stride, pad):
    r = gen.rng(B + Cin + Tin)
    x = gen.i8(r, (B, Cin, Tin))
    w = gen.i8(r, (Cout, Cin * ks))
    bias = r.integers(-2**31, 2**31, size=Cout, dtype=np.int64).astype(np.int32)
    for mult, shift in ((0x80000000, 0), (int(r.integers(0, 2**32)), 7), (5, -9), (2**32 - 1, 40)):
        assert np.array_equal(oracle.conv1d(x, w, bias, mult, shift, stride, pad),
                              ref.conv1d(x, w, bias, mult, shift, stride, pad))
        assert np.array_equal(oracle.conv1d(x, w, None, mult, shift, stride, pad),
                              ref.conv1d(x, w, None, mult, shift, stride, pad))


def test_classifier_vs_ref(oracle, ref):
    r = gen.rng(6)
    x = gen.i8(r, (1, 3, 40))
    w = gen.i8(r, (257, 40))
    for mult, shift in ((0x80000000, 0), (int(r.integers(0, 2**32)), 3), (7, -2), (1, 33)):
        assert np.array_equal(oracle.classifier(x, w, mult, shift), ref.classifier(x, w, mult, shift))


ATT = [(1, 1, 1, 1, 1), (1, 2, 3, 5, 4), (2, 3, 4, 4, 16), (1, 1, 1, 33, 64), (2, 2, 7, 9, 17),
       (1, 2, 16, 16, 64)]


@pytest.mark.parametrize("B,H,Tq,Tk,D", ATT)
@pytest.mark.parametrize("masked", [False, True])
def test_attention_vs_ref(oracle, ref, B, H, Tq, Tk, D, masked):
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(B + H + Tq + Tk + D, B, H, Tq, Tk, D)
    mask = gen.causal_mask(Tq, Tk) if masked and Tk >= Tq else None
    for (qm_, qs_, f_, am_, as__) in ((qm, qs, f, am, as_), (255, -3, 1, 1, 40), (1, 40, 13, 255, -2),
                                      (200, 0, 8, 17, 0)):
        a = oracle.qk_requant_rowmax(q, k, mask, qm_, qs_)
        b = ref.qk_requant_rowmax(q, k, mask, qm_, qs_)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        pa = oracle.shift_exp(a[0], a[1], mask, f_)
        pb = ref.shift_exp(b[0], b[1], mask, f_)
        assert np.array_equal(pa[0], pb[0]) and np.array_equal(pa[1], pb[1])
        for off in (16, 0, 29):
            assert np.array_equal(oracle.pv_norm_requant(pa[0], v, pa[1], am_, as__, off),
                                  ref.pv_norm_requant(pb[0], v, pb[1], am_, as__, off))


def test_shift_exp_all_inputs_vs_ref(oracle, ref):
    """Every int16 score against every row max class, for every legal frac_bits."""
    qk = np.arange(-32768, 32768, dtype=np.int16).reshape(1, 1, 1, -1)
    for f in range(1, 14):
        for rm in (-32768, -32767, -1, 0, 1, 300, 32767):
            rmx = np.array([[[[rm]]]], np.int16)
            a = oracle.shift_exp(qk, rmx, None, f)
            b = ref.shift_exp(qk, rmx, None, f)
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_shift_exp_table_clamp_is_exact(oracle):
    """The fused attention kernels map a score to P through a 32768-entry table
    indexed by min((row_max + 1 - score) mod 2^16, 32767). That equals the
    reference's shift-exponential of every int16 difference, for every legal
    frac_bits, because P is 0 from index 22796 on (and for the positive
    differences above 32768 that the int16 wrap produces)."""
    qk = np.arange(-32768, 32768, dtype=np.int16).reshape(1, 1, 1, -1)
    zero = np.zeros((1, 1, 1, 1), np.int16)
    for f in range(1, 14):
        p = oracle.shift_exp(qk, zero, None, f)[0].reshape(-1)  # p[x + 32768] = P(x - 0)
        table = p[32768 - np.arange(32768)]                      # table[i] = P(-i)
        idx = (-qk.reshape(-1).astype(np.int64)) & 0xFFFF
        assert np.array_equal(table[np.minimum(idx, 32767)], p), f
        assert not table[22796:].any(), f


def test_pv_negative_row_sum_raises(oracle, ref):
    p = np.zeros((1, 1, 1, 4), np.uint8)
    v = np.zeros((1, 1, 2, 4), np.int8)
    rs = np.array([[[[-1]]]], np.int32)
    for impl in (oracle, ref):
        with pytest.raises(ValueError):
            impl.pv_norm_requant(p, v, rs, 1, 0, 16)


# ---------------------------------------------------------------------------
# 3. known answers and closed forms (no reference build needed)
# ---------------------------------------------------------------------------

def test_linear_accum_known_answers(oracle):
    """Hand-computed values from tests/kernels/test_linear8_scalar.py:103-260 of the reference."""
    x = np.array([[1, 2, 3], [-1, 4, 2]], np.int8)
    w = np.array([[1, 0, -1], [2, 1, 3]], np.int8)
    assert oracle.linear_accum(x, w, None, None).tolist() == [[-2, 13], [-3, 8]]
    assert oracle.linear_accum(x, w, np.array([10, -5], np.int32), None).tolist() == [[8, 8], [7, 3]]
    # zero point: acc - wz[n] * rowsum(x), rowsums 6 and 5
    got = oracle.linear_accum(x, w, None, np.array([2, -1], np.int8))
    assert got.tolist() == [[-2 - 12, 13 + 6], [-3 - 10, 8 + 5]]


def test_linear_accum_matches_int64_matmul(oracle):
    r = gen.rng(10)
    for M, K, N in ((5, 1280, 7), (3, 5120, 4), (17, 33, 9)):
        x, w, b, z, _, _ = gen.linear_case(M + K, M, K, N)
        exact = (x.astype(np.int64) @ w.astype(np.int64).T + b.astype(np.int64)
                 - z.astype(np.int64)[None, :] * x.astype(np.int64).sum(1, keepdims=True))
        wrapped = ((exact + 2**31) % 2**32 - 2**31).astype(np.int32)
        assert np.array_equal(oracle.linear_accum(x, w, b, z), wrapped)


def _rshift_closed(x, s):
    """Round half away from zero of x / 2^s (the s == 0 / s >= 32 cases of fixedpoint.h:64-70)."""
    if s == 0:
        return x
    if s >= 32:
        return 0
    q = (abs(x) + (1 << (s - 1))) >> s
    return q if x >= 0 else -q


def test_rshift_closed_form(oracle):
    r = gen.rng(11)
    xs = list(r.integers(-2**31, 2**31 - 2**20, 3000)) + [0, 1, -1, 2, -2, 3, -3, 6, 7, -6, -7]
    for x in xs:
        for s in (0, 1, 2, 5, 15, 30, 31, 32, 40):
            x = int(x)
            if 0 < s < 32 and x + (1 << (s - 1)) >= 2**31:
                # the rounding add wraps modulo 2^32 (fixedpoint.h:72-86)
                assert oracle.rshift(x, s) == (x + (1 << (s - 1)) - 2**32) >> s, (x, s)
            else:
                assert oracle.rshift(x, s) == _rshift_closed(x, s), (x, s)


def test_rshift_boundaries_from_reference_tests(oracle):
    """tests/kernels/test_linear8_scalar.py:759-800: accum 2,3,-2,-3 >> 1 and 6,7,-6,-7 >> 2
    after mulh by 0x80000000 (i.e. halving)."""
    acc = [2, 3, -2, -3, 6, 7, -6, -7]
    sh = [1, 1, 1, 1, 2, 2, 2, 2]
    got = [oracle.requant(a, 0x80000000, s) for a, s in zip(acc, sh)]
    exp = [_rshift_closed(math.floor(a / 2), s) for a, s in zip(acc, sh)]
    assert got == exp


def test_mulh_closed_form(oracle):
    r = gen.rng(12)
    for _ in range(3000):
        x = int(r.integers(-2**31, 2**31))
        m = int(r.integers(0, 2**32))
        assert oracle.mulh(x, m) == (x * m) >> 32
    for x, m in ((100, 0x80000000), (-100, 0x80000000), (1234567, 0x40000000), (-1, 0xFFFFFFFF)):
        assert oracle.mulh(x, m) == (x * m) >> 32


def test_fisr_approximates_inverse_sqrt(oracle):
    """FISR(x, off) ~ 2^off / sqrt(x) within the integer truncation error (< 2 %)."""
    # Domains the path uses: LayerNorm variances (offset 13) and attention row
    # sums (offset 16, at least one P of 95 per row). Below them the
    # reference's int32 Newton steps wrap (kept bit-exact by the differential
    # tests above).
    for off, lo in ((13, 64), (16, 95)):
        for x in list(range(lo, 300000, 3)) + [10**6, 10**8]:
            y = oracle.fisr(x, off)
            ideal = 2**off / math.sqrt(x)
            if ideal >= 16:
                assert abs(y - ideal) / ideal < 0.035, (off, x, y, ideal)


def test_shift_exp_closed_form(oracle):
    """For x_sub in [-2^f * 4, 0] no int16 wrap occurs and P is
    ((2^f + (frac >> 1)) >> -xi) >> (f - 7) with fix = x + (x>>1) - (x>>4)."""
    for f in range(1, 14):
        lo = max(-(4 << f), -20000)
        for x in range(lo, 1):
            fix = x + (x >> 1) - (x >> 4)
            xi = fix >> f
            frac = fix - xi * (1 << f)
            num = (1 << f) + (frac >> 1)
            e = 0 if -xi >= 16 else num >> (-xi)
            p = (e >> (f - 7)) if f > 7 else e
            assert oracle.shift_exp_one(x, f) == (p & 0xFF), (f, x)
        assert oracle.shift_exp_one(5, f) == 0


def test_shift_exp_table_tail_is_zero(oracle):
    """The fused kernel folds every x_sub <= -32767 and every x_sub > 0 onto one
    zero table entry; this holds for every legal frac_bits."""
    for f in range(1, 14):
        assert oracle.shift_exp_one(-32767, f) == 0
        assert oracle.shift_exp_one(-32768, f) == 0
        assert max(oracle.shift_exp_one(-i, f) for i in range(1, 32768, 97)) <= 127
        assert oracle.shift_exp_one(0, f) == min(1 << f, 128) % 256


def test_elementwise_brute_force(oracle):
    """GeLU, residual15 and add_requant15 over every int8 input against closed forms."""
    x = np.arange(-128, 128, dtype=np.int8).reshape(1, -1)
    lut = np.arange(0, 256, 16, dtype=np.uint8)
    for im, is_, om, os_ in ((3, 2, 5, 6), (255, 13, 1, 0), (1, 0, 255, 20)):
        got = oracle.gelu(x, lut, np.array([im], np.uint8), np.array([is_], np.int8),
                          np.array([om], np.uint8), np.array([os_], np.int8))
        for v, g in zip(x[0].astype(int), got[0].astype(int)):
            idx = min(max(_rshift_closed(v * im, is_) + 8, 0), 15)
            y = _rshift_closed(v * int(lut[idx]) * om, os_)
            assert g == min(max(y, -127), 127)
    res = np.arange(-128, 128, dtype=np.int16) * 100
    br = np.arange(256, dtype=np.int32) * 77777 - 9000000
    got = oracle.residual15(br, res, 300)
    for b_, r_, g in zip(br.astype(int), res.astype(int), got.astype(int)):
        assert g == min(max(_rshift_closed(b_ + r_ * 300, 15), -16383), 16383)


def test_layernorm_invariants(oracle):
    """Mean of a constant row is the constant for widths that divide exactly
    (512, 1024); a constant row normalises to beta-only output."""
    for h in (512, 1024):
        x = np.full((2, h), 1234, np.int16)
        g = np.full(h, 10, np.int8)
        b = np.arange(h, dtype=np.int32)
        out = oracle.layernorm32(x, g, b, 128, 10, 0x80000000, 0)
        exp = np.clip([_rshift_closed((int(v) * 0x80000000) >> 32, 0) for v in b], -127, 127)
        assert np.array_equal(out[0], np.array(exp, np.int8))


def test_model_oracle_cached_steps_equal_one_causal_pass(iw):
    """The decoder over the cache, one token per step (model_int.py:1398-1442 with
    the hook cache of :1587-1618), gives at every step the logits that one causal
    pass over the whole token sequence gives at that position (the mask slice
    mask[k_len - q_len : k_len, :k_len] of model_int.py:794-797 leaves query t
    the keys 0 .. t either way). The workload parity tests rely on this."""
    from oracle.model_oracle import OracleWhisper

    dims = iw.ModelDimensions(n_mels=80, n_audio_ctx=40, n_audio_state=384, n_audio_head=6,
                              n_audio_layer=1, n_vocab=300, n_text_ctx=24, n_text_state=384,
                              n_text_head=6, n_text_layer=2)
    P = iw.synth.calibrated_int_params(dims, seed=8, decoder_mlp_scale=0.1)
    o = OracleWhisper(dims, P, threads=4)
    xa = o.encoder(iw.synth.synthetic_mel(2, 80, 80, seed=9))
    prompt = np.array([[5, 17, 200], [9, 9, 31]], np.int64)
    toks, step_logits = o.greedy(xa, prompt, 10, return_logits=True)
    full = o.decoder_logits(toks[:, :-1], xa)
    assert np.array_equal(full[:, 2:], step_logits)
    # teacher forcing through the cache agrees with the causal pass as well
    forced = np.random.default_rng(3).integers(0, 300, size=(2, 9))
    f_argmax, f_logits = o.forced(xa, prompt, forced)
    full = o.decoder_logits(np.concatenate([prompt, forced], 1), xa)
    assert np.array_equal(full[:, 2:], f_logits)
    assert np.array_equal(f_argmax, full[:, 2:].argmax(-1))
