"""The SIMD-shaped CPU baseline (oracle/iw_cpu_simd.c: int8 dot-product tiles
split over threads, as the reference's CPU backend runs its kernels) is
bit-identical to the scalar oracle on every op it implements, including
K / N tails, M below and above the tile-shape thresholds, masked attention,
and a whole model."""
import numpy as np
import pytest

from tests import gen


@pytest.fixture(scope="module")
def simd():
    from oracle.oracle import Oracle, available, build

    if not available("simd"):
        build()
    return Oracle("simd", threads=4)


@pytest.mark.parametrize("M,K,N", [(1, 1280, 33), (3, 100, 7), (17, 384, 64), (64, 131, 258), (40, 2048, 96)])
def test_linear_matches_oracle(oracle, simd, M, K, N):
    r = gen.rng(M * 7 + K + N)
    x = gen.i8(r, (M, K))
    w = gen.i8(r, (N, K))
    b = r.integers(-2**31, 2**31, N).astype(np.int32)
    z = gen.i8(r, (N,))
    m = r.integers(0, 2**32, N, dtype=np.uint64).astype(np.uint32)
    s = r.integers(-3, 40, N).astype(np.int8)
    for bias, wz in ((b, z), (None, None), (b, None)):
        assert np.array_equal(simd.linear8(x, w, bias, wz, m, s), oracle.linear8(x, w, bias, wz, m, s))
        assert np.array_equal(simd.linear32(x, w, bias, wz, m, s), oracle.linear32(x, w, bias, wz, m, s))


def test_classifier_and_conv_match_oracle(oracle, simd):
    r = gen.rng(9)
    x = gen.i8(r, (2, 3, 384))
    w = gen.i8(r, (1001, 384))
    for mult, shift in ((0x9e3779b9, 12), (0x80000000, -2), (5, 40)):
        assert np.array_equal(simd.classifier(x, w, mult, shift), oracle.classifier(x, w, mult, shift))
    xc = gen.i8(r, (2, 80, 61))
    for cout, stride in ((40, 1), (36, 2)):
        wc = gen.i8(r, (cout, 80 * 3))
        bc = r.integers(-50000, 50000, cout).astype(np.int32)
        assert np.array_equal(simd.conv1d(xc, wc, bc, 0x7fff1234, 9, stride, 1),
                              oracle.conv1d(xc, wc, bc, 0x7fff1234, 9, stride, 1))


@pytest.mark.parametrize("Tq,Tk,D,masked", [(1, 1500, 64, False), (37, 37, 64, True), (20, 50, 96, False),
                                            (5, 130, 128, True)])
def test_attention_matches_oracle(oracle, simd, Tq, Tk, D, masked):
    r = gen.rng(Tq + Tk + D)
    B, H = 2, 3
    q = gen.i8(r, (B, H, Tq, D))
    k = gen.i8(r, (B, H, Tk, D))
    v = gen.i8(r, (B, H, D, Tk))
    mask = np.triu(np.ones((Tq, Tk), bool), Tk - Tq + 1) if masked else None
    args = (q, k, v, mask, 97, 9, 8, 201, 7, 16)
    assert np.array_equal(simd.attention(*args), oracle.attention(*args))


def test_whole_model_matches_oracle(iw):
    from oracle.model_oracle import OracleWhisper

    dims = iw.ModelDimensions(n_mels=80, n_audio_ctx=40, n_audio_state=384, n_audio_head=6, n_audio_layer=1,
                              n_vocab=300, n_text_ctx=24, n_text_state=384, n_text_head=6, n_text_layer=1)
    P = iw.synth.calibrated_int_params(dims, seed=3)
    mel = iw.synth.synthetic_mel(1, 80, 80, seed=4)
    a, b = OracleWhisper(dims, P, threads=4), OracleWhisper(dims, P, threads=4, kind="simd")
    xa = a.encoder(mel)
    assert np.array_equal(b.encoder(mel), xa)
    prompt = np.array([[1, 2, 3]], np.int64)
    assert np.array_equal(b.greedy(xa, prompt, 6, return_logits=True)[1], a.greedy(xa, prompt, 6, return_logits=True)[1])


def test_avx2_path_matches_oracle(oracle):
    """The AVX2 dot tiles (the path taken where AVX-512 VNNI is absent)."""
    import ctypes as C

    from oracle.oracle import Oracle

    s = Oracle("simd", threads=2)
    s.lib.iws_force_isa.argtypes = [C.c_int]
    s.lib.iws_force_isa(0)
    try:
        r = gen.rng(5)
        x, w = gen.i8(r, (33, 77)), gen.i8(r, (10, 77))
        m = np.full(10, 0x70000000, np.uint32)
        sh = np.full(10, 5, np.int8)
        assert np.array_equal(s.linear8(x, w, None, None, m, sh), oracle.linear8(x, w, None, None, m, sh))
        q, k, v = gen.i8(r, (1, 2, 9, 64)), gen.i8(r, (1, 2, 9, 64)), gen.i8(r, (1, 2, 64, 9))
        args = (q, k, v, None, 50, 6, 7, 150, 6, 16)
        assert np.array_equal(s.attention(*args), oracle.attention(*args))
    finally:
        s.lib.iws_force_isa(-1)
