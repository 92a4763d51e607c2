"""Bit-exact parity of the decode-step entry points (KV-cache layouts, device-side
cache position, graph replay) against the CPU oracle.

* iw_attention_decode_cache: one query row per (batch, head) over per-head
  caches with garbage past the valid keys; the key count is k_length + *pos,
  clamped to max_keys.
* iw_linear8_qkv_cache: the QKV projection appending K / V at *pos.
* iw_embed_tokens / iw_greedy_advance: the embedding and greedy bookkeeping
  of a step whose position lives on the device.
* A captured decode step replayed many times gives the eager tokens.
"""
import numpy as np
import pytest
import torch

from tests import gen

pytestmark = pytest.mark.gpu


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


T_ = T


def host(t):
    return t.cpu().numpy()


def stream():
    return torch.cuda.current_stream().cuda_stream


def _decode_cache(iw, q, k, v, qm, qs, f, am, as_, *, tcap, k_length, pos_val, max_keys, layout="vt"):
    """q [B,H,1,D], k [B,H,Tk,D], v [B,H,D,Tk] placed in caches with random fill
    (V in the given cache layout)."""
    B, H, _, D = q.shape
    Tk = k.shape[2]
    r = gen.rng(B + H + Tk)
    kc = gen.i8(r, (B, H, tcap, D))
    kc[:, :, :Tk] = k
    shape, vs = gen.v_cache_layout(B, H, D, tcap, layout)
    vc = gen.i8(r, shape)
    gen.v_cache_put(vc, layout, 0, v)
    qh = np.ascontiguousarray(q[:, :, 0, :].reshape(B, H * D))
    out = torch.empty((B, H * D), dtype=torch.int8, device="cuda")
    pos = None if pos_val is None else torch.tensor([pos_val], dtype=torch.int32, device="cuda")
    qt, kt, vt = T(qh), T(kc), T(vc)
    iw._lib.call("iw_attention_decode_cache", qt.data_ptr(), H * D, kt.data_ptr(), H * tcap * D,
                 tcap * D, D, vt.data_ptr(), *vs, out.data_ptr(), H * D, B, H,
                 D, k_length, None if pos is None else pos.data_ptr(), max_keys, qm, qs, f, am, as_, 16,
                 stream())
    return host(out).reshape(B, 1, H * D)


# V in key quads is read for head_dim 64 only (test_attention_decode_cache_quads_rejects
# checks the refusal); head_dim 96 and 128 run with V transposed
_DECODE_CASES = [(2, 3, 64, 1, 448, 1), (2, 3, 64, 17, 448, 1), (1, 2, 64, 448, 448, 1), (3, 2, 64, 200, 448, 1),
                 (2, 4, 64, 1500, 1500, 1500), (2, 2, 64, 33, 40, 33)]


@pytest.mark.parametrize("B,H,D,Tk,tcap,k_length,layout",
                         [c + (lay,) for c in _DECODE_CASES for lay in gen.V_LAYOUTS]
                         + [(1, 2, 96, 100, 448, 1, "vt"), (1, 1, 128, 300, 448, 1, "vt")])
def test_attention_decode_cache(iw, oracle, gpu, B, H, D, Tk, tcap, k_length, layout):
    print("case: decode cache", B, H, D, Tk, tcap, k_length, layout, flush=True)
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(3 * B + Tk + D, B, H, 1, Tk, D)
    exp = oracle.attention(q, k, v, None, qm, qs, f, am, as_)
    pos_val = None if k_length == Tk else Tk - k_length
    got = _decode_cache(iw, q, k, v, qm, qs, f, am, as_, tcap=tcap, k_length=k_length,
                        pos_val=pos_val, max_keys=tcap if pos_val is not None else k_length, layout=layout)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("Tk", [1, 2, 3, 4, 5, 127, 128, 129, 255, 257, 446, 447, 448])
def test_attention_decode_cache_quads_ragged(iw, oracle, gpu, Tk):
    """Key counts that end inside a quad, a 128-key chunk or the cache
    (self-attention shapes: 20 heads, 448 positions, key count k_length + *pos)."""
    print("case: decode cache quads ragged", Tk, flush=True)
    B, H, D, tcap = 3, 20, 64, 448
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(31 * Tk + 5, B, H, 1, Tk, D)
    exp = oracle.attention(q, k, v, None, qm, qs, f, am, as_)
    got = _decode_cache(iw, q, k, v, qm, qs, f, am, as_, tcap=tcap, k_length=1, pos_val=Tk - 1,
                        max_keys=tcap, layout="quads")
    assert np.array_equal(got, exp)


def test_attention_decode_cache_quads_rejects(iw, gpu):
    """Key quads need head_dim 64, v_sd 4 and a 16-byte multiple v_sq of at
    least 4 head_dim."""
    B, H, tcap = 1, 2, 64
    q = torch.zeros((B, H * 96), dtype=torch.int8, device="cuda")
    k = torch.zeros((B, H, tcap, 96), dtype=torch.int8, device="cuda")
    v = torch.zeros(B * H * tcap * 96 + 4096, dtype=torch.int8, device="cuda")
    out = torch.empty((B, H * 96), dtype=torch.int8, device="cuda")
    for D, vs, what in ((96, (H * tcap * 96, tcap * 96, 4, 384), "head_dim 64"),
                        (64, (H * tcap * 64, tcap * 64, 4, 240), "v_sq >= 4"),
                        (64, (H * tcap * 64, tcap * 64, 4, 264), "v_sq % 16"),
                        (64, (H * tcap * 64, tcap * 64, 8, 256), "v_sd == 4")):
        with pytest.raises(RuntimeError, match=what):
            iw._lib.call("iw_attention_decode_cache", q.data_ptr(), H * D, k.data_ptr(), H * tcap * D, tcap * D,
                         D, v.data_ptr(), *vs, out.data_ptr(), H * D, B, H, D, 1, None, 1, 1, 1, 8, 1, 1, 16,
                         stream())


@pytest.mark.parametrize("layout", ["vt", "quads"])
def test_attention_decode_cache_clamps_keys(iw, oracle, gpu, layout):
    """A device position past the cache reads max_keys keys, not beyond."""
    B, H, D, tcap = 1, 2, 64, 64
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(77, B, H, 1, tcap, D)
    exp = oracle.attention(q, k, v, None, qm, qs, f, am, as_)
    got = _decode_cache(iw, q, k, v, qm, qs, f, am, as_, tcap=tcap, k_length=1, pos_val=10_000,
                        max_keys=tcap, layout=layout)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("layout", ["vt", "quads"])
def test_attention_decode_cache_wrap_corner(iw, oracle, gpu, layout):
    B, H, D, Tk = 1, 1, 64, 40
    q = np.full((B, H, 1, D), 127, np.int8)
    k = np.full((B, H, Tk, D), 127, np.int8)
    k[..., 1::3, :] = -128
    v = gen.i8(gen.rng(1), (B, H, D, Tk))
    exp = oracle.attention(q, k, v, None, 255, 0, 8, 200, 6)
    got = _decode_cache(iw, q, k, v, 255, 0, 8, 200, 6, tcap=448, k_length=1, pos_val=Tk - 1,
                        max_keys=448, layout=layout)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("layout", ["vt", "quads"])
@pytest.mark.parametrize("wrap_head", [0, 1])
@pytest.mark.parametrize("B,H,Tk,tcap", [(1, 2, 700, 1024), (3, 4, 1500, 1500), (2, 2, 40, 448)])
def test_attention_decode_cache_heads_share_a_block(iw, oracle, gpu, wrap_head, B, H, Tk, tcap, layout):
    """Cross-attention-sized caches run two heads per block as one stream: each
    head's row maximum, P, sums and wrap flag must stay its own. One head of
    every pair takes the int16 row-max wrap (P = 128), the other does not."""
    print("case: heads share a block", wrap_head, B, H, Tk, tcap, layout, flush=True)
    D = 64
    q, k, v, qm, qs, f, am, as_ = gen.attn_case(11 * B + H + Tk, B, H, 1, Tk, D)
    for h in range(wrap_head, H, 2):
        q[:, h] = 127
        k[:, h] = 127
        k[:, h, 1::3] = -128
    qm, qs, f = 255, 0, 8
    exp = oracle.attention(q, k, v, None, qm, qs, f, am, as_)
    got = _decode_cache(iw, q, k, v, qm, qs, f, am, as_, tcap=tcap, k_length=Tk, pos_val=None, max_keys=Tk,
                        layout=layout)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("B,Tn,H,D,pos_val,tcap", [(1, 1, 2, 64, 0, 448), (5, 1, 2, 64, 7, 448),
                                                    (128, 1, 2, 64, 100, 448), (4, 3, 2, 64, 0, 448),
                                                    (2, 3, 4, 32, 38, 40), (40, 3, 2, 64, 5, 448),
                                                    (3, 3, 2, 64, 446, 448)])
@pytest.mark.parametrize("layout", gen.V_LAYOUTS)
def test_linear8_qkv_cache(iw, oracle, gpu, B, Tn, H, D, pos_val, tcap, layout):
    print("case: qkv cache", B, Tn, H, D, pos_val, tcap, layout, flush=True)
    C = H * D
    M = B * Tn
    x, w, b, z, m, s = gen.realistic_linear_case(M + C + pos_val, M, C, 3 * C)
    exp = oracle.linear8(x, w, b, z, m, s)
    r = gen.rng(5)
    kc0 = gen.i8(r, (B, H, tcap, D))
    shape, vs = gen.v_cache_layout(B, H, D, tcap, layout)
    vc0 = gen.i8(r, shape)
    kc, vc = T(kc0), T(vc0)
    q = torch.empty((M, C), dtype=torch.int8, device="cuda")
    pos = torch.tensor([pos_val], dtype=torch.int32, device="cuda")
    xt, wt, bt, zt, mt, st = T(x), T(w), T(b), T(z), T(m), T(s)  # alive across the call
    iw._lib.call("iw_linear8_qkv_cache", xt.data_ptr(), wt.data_ptr(), bt.data_ptr(), zt.data_ptr(),
                 mt.data_ptr(), st.data_ptr(), M, C, True, True, q.data_ptr(), C,
                 kc.data_ptr(), H * tcap * D, tcap * D, D, vc.data_ptr(), *vs,
                 C, D, Tn, tcap, pos.data_ptr(), stream())
    torch.cuda.synchronize()
    assert np.array_equal(host(q), exp[:, :C])
    kexp, vexp = kc0.copy(), vc0.copy()
    e = exp.reshape(B, Tn, 3, H, D)
    for i in range(Tn):
        t = pos_val + i
        if t < tcap:
            kexp[:, :, t, :] = e[:, i, 1]
            gen.v_cache_put(vexp, layout, t, e[:, i, 2][..., None])
    assert np.array_equal(host(kc), kexp)
    assert np.array_equal(host(vc), vexp)


@pytest.mark.parametrize("B,T,H,D,t_off", [(2, 1500, 4, 64, 0), (1, 37, 2, 64, 16), (3, 64, 3, 32, 0),
                                           (2, 100, 2, 64, 3), (1, 5, 2, 48, 0)])
@pytest.mark.parametrize("layout", gen.V_LAYOUTS)
def test_transpose_heads(iw, gpu, B, T, H, D, t_off, layout):
    """V of a fused [B, T, 3C] projection into a per-head V cache (transposed
    rows or key quads) at positions t_off .. t_off + T; every other byte is
    left as it was."""
    print("case: transpose heads", B, T, H, D, t_off, layout, flush=True)
    C = H * D
    r = gen.rng(T + t_off)
    qkv = gen.i8(r, (B, T, 3 * C))
    tcap = (t_off + T + 15) // 16 * 16 + 16
    shape, vs = gen.v_cache_layout(B, H, D, tcap, layout)
    dst0 = np.full(shape, 0x55, np.int8)
    src, dst = T_(qkv), T_(dst0)
    iw._lib.call("iw_transpose_heads", src.data_ptr() + 2 * C, T * 3 * C, 3 * C, dst.data_ptr(), *vs,
                 t_off, B, T, H, D, stream())
    torch.cuda.synchronize()
    exp = dst0.copy()
    gen.v_cache_put(exp, layout, t_off, qkv[:, :, 2 * C:].reshape(B, T, H, D).transpose(0, 2, 3, 1))
    assert np.array_equal(host(dst), exp)


def test_embed_tokens(iw, oracle, gpu):
    r = gen.rng(11)
    B, V, C, n_ctx = 6, 500, 128, 40
    table = gen.i8(r, (V, C))
    pe = gen.i8(r, (n_ctx, C))
    tokens = r.integers(0, V, size=B).astype(np.int64)
    m16 = np.array([int(r.integers(1, 65536))], np.uint16)
    s8 = np.array([9], np.int8)
    tt, tab, pet, mt, st = T(tokens), T(table), T(pe), T(m16), T(s8)  # alive across the calls
    for pos_val in (0, 17, n_ctx - 1, n_ctx + 5):
        pos = torch.tensor([pos_val], dtype=torch.int32, device="cuda")
        out = torch.empty((B, C), dtype=torch.int16, device="cuda")
        iw._lib.call("iw_embed_tokens", tt.data_ptr(), tab.data_ptr(), pet.data_ptr(), n_ctx,
                     pos.data_ptr(), mt.data_ptr(), st.data_ptr(), out.data_ptr(), B, C, stream())
        p = min(pos_val, n_ctx - 1)  # a position past the table reads its last row
        exp = oracle.add_requant15(table[tokens][:, None, :], pe[p:p + 1], m16, s8)
        assert np.array_equal(host(out), exp[:, 0])


def test_greedy_advance(iw, gpu):
    r = gen.rng(12)
    B, V, cols = 5, 1000, 4
    hist = torch.full((B, cols), -1, dtype=torch.int64, device="cuda")
    nxt = torch.empty(B, dtype=torch.int64, device="cuda")
    step = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos = torch.tensor([3], dtype=torch.int32, device="cuda")
    rows = []
    for i in range(cols + 1):
        lg = gen.i8(r, (B, V))
        lg[0, 10] = lg[0, 20] = 127  # first maximum wins
        lgt = T(lg)
        iw._lib.call("iw_greedy_advance", lgt.data_ptr(), B, V, V, nxt.data_ptr(), hist.data_ptr(),
                     cols, cols, step.data_ptr(), pos.data_ptr(), 1 if i else 3, stream())
        assert np.array_equal(host(nxt), np.argmax(lg, 1))
        rows.append(np.argmax(lg, 1))
    assert np.array_equal(host(hist), np.stack(rows[:cols], 1))  # the extra step is not recorded
    assert int(step.item()) == cols + 1 and int(pos.item()) == 3 + 3 + cols


def test_gather_heads(iw, gpu):
    r = gen.rng(13)
    B, Tn, H, D, tcap, off = 3, 7, 4, 32, 20, 5
    src = gen.i8(r, (B, Tn, 3, H * D))
    dst0 = gen.i8(r, (B, H, tcap, D))
    dst = T(dst0)
    st = T(src)
    iw._lib.call("iw_gather_heads", st.data_ptr() + H * D, Tn * 3 * H * D, 3 * H * D, dst.data_ptr(),
                 H * tcap * D, tcap * D, D, off, B, Tn, H, D, stream())
    exp = dst0.copy()
    exp[:, :, off:off + Tn, :] = src[:, :, 1].reshape(B, Tn, H, D).transpose(0, 2, 1, 3)
    assert np.array_equal(host(dst), exp)


@pytest.fixture(scope="module")
def tiny_model(iw):
    dims = iw.ModelDimensions(n_mels=80, n_audio_ctx=50, n_audio_state=384, n_audio_head=6,
                              n_audio_layer=1, n_vocab=300, n_text_ctx=24, n_text_state=384,
                              n_text_head=6, n_text_layer=2)
    params = iw.synth.calibrated_int_params(dims, seed=99, calib_ctx=50)
    return dims, params


def test_graph_replay_matches_eager_and_oracle(iw, gpu, tiny_model):
    """The captured one-token step, replayed across two utterances, gives the eager
    tokens and the oracle's."""
    from oracle.model_oracle import OracleWhisper

    dims, params = tiny_model
    model = iw.Whisper_int.from_params(dims, params).cuda()
    ref = OracleWhisper(dims, params, threads=4)
    B, steps = 3, 12
    runner = iw.DecoderRunner(model.decoder, B, dims.n_audio_ctx, use_graph=True)
    for seed in (1, 2):
        mel = iw.synth.synthetic_mel(B, dims.n_mels, 2 * dims.n_audio_ctx, seed=seed)
        prompt = np.random.default_rng(seed).integers(0, dims.n_vocab, size=(B, 3)).astype(np.int64)
        with torch.no_grad():
            feats = model.embed_audio(T(mel))
            g_toks = iw.greedy_decode(model, feats, T(prompt), steps, runner=runner)
            e_toks, _ = iw.greedy_decode(model, feats, T(prompt), steps, keep_logits=True)
        torch.cuda.synchronize()
        assert np.array_equal(host(g_toks), host(e_toks)), f"utterance {seed}"
        r_toks = ref.greedy(ref.encoder(mel), prompt, steps)
        assert np.array_equal(host(g_toks), r_toks), f"utterance {seed}"


def test_weight_prefetch_does_not_change_results(iw, gpu, tiny_model):
    """The one-token step with and without the next-GEMM weight prefetch (the
    LayerNorms and FC1 reading the next GEMM's weight tiles into L2): the same
    greedy tokens, replayed from graphs of 8 steps and of one step, and the
    same logits step by step."""
    dims, params = tiny_model
    model = iw.Whisper_int.from_params(dims, params).cuda()
    # 18 steps after the prompt: one eager warm-up step before capture, two
    # replays of the 8-step graph and one replay of the one-step graph
    B, steps = 5, 19
    mel = iw.synth.synthetic_mel(B, dims.n_mels, 2 * dims.n_audio_ctx, seed=7)
    prompt = np.random.default_rng(7).integers(0, dims.n_vocab, size=(B, 3)).astype(np.int64)
    runners = [iw.DecoderRunner(model.decoder, B, dims.n_audio_ctx, prefetch=pf) for pf in (False, True)]
    eager = [iw.DecoderRunner(model.decoder, B, dims.n_audio_ctx, use_graph=False, prefetch=pf)
             for pf in (False, True)]
    with torch.no_grad():
        feats = model.embed_audio(T(mel))
        toks = [host(iw.greedy_decode(model, feats, T(prompt), steps, runner=r)) for r in runners]
        logits = [host(iw.greedy_decode(model, feats, T(prompt), steps, runner=r, keep_logits=True)[1])
                  for r in eager]
    assert np.array_equal(toks[0], toks[1])
    assert np.array_equal(logits[0], logits[1])


def _unfrag(img, rows, cols):
    """Row-major [rows, cols] from a fragment-major image (iwhisper_amd.h layout)."""
    kp = (cols + 319) // 320 * 320
    r = np.arange(rows)[:, None]
    k = np.arange(cols)[None, :]
    off = (r // 32) * 32 * kp + (k // 32) * 1024 + (r % 32 + 32 * ((k // 16) % 2)) * 16 + k % 16
    return img[off]


@pytest.mark.parametrize("B,H,Tk,bias,asym", [(2, 20, 1500, True, True), (5, 6, 1500, True, True),
                                             (3, 12, 100, False, True), (1, 16, 7, True, False),
                                             (128, 20, 1500, True, True)])
def test_attention_decode_cross_lnq(iw, oracle, gpu, B, H, Tk, bias, asym):
    """The cross-attention with the LayerNorm and query projection fused in
    against the oracle chain layernorm32 -> linear8 -> attention: one row with
    the full int16 range (|x - mean| > 46340: the per-element variance form),
    query shifts outside [0, 31], every supported width."""
    print("case: cross_lnq", B, H, Tk, bias, asym, flush=True)
    D = 64
    C = H * D
    x, gamma, beta, lm, ls, om, os_ = gen.ln_case(B * 7 + H + Tk, B, C)
    x[0, ::2], x[0, 1::2] = 32767, -32768
    _, w, qb, qz, qm_, qs_ = gen.realistic_linear_case(B + C + Tk, 1, C, C, has_bias=bias, asym=asym)
    qs_[:2] = [-1, 32]
    q_, k, v, qm, qs, f, am, as_ = gen.attn_case(B + H + Tk + 1, B, H, 1, Tk, D)
    h8 = oracle.layernorm32(x, gamma, beta, lm, ls, om, os_, 13)
    q8 = oracle.linear8(h8, w, qb, qz, qm_, qs_)
    exp = oracle.attention(np.ascontiguousarray(q8.reshape(B, 1, H, D).transpose(0, 2, 1, 3)), k, v, None, qm, qs,
                           f, am, as_)
    t16 = (Tk + 15) // 16 * 16
    vt = np.zeros((B, H, D, t16), np.int8)
    vt[..., :Tk] = v
    wf = torch.zeros(iw._lib.value("iw_frag_bytes", C, C), dtype=torch.int8, device="cuda")
    wt = T(w)
    iw._lib.call("iw_frag_pack", wt.data_ptr(), C, C, C, wf.data_ptr(), stream())
    out = torch.zeros(iw._lib.value("iw_frag_bytes", B, C), dtype=torch.int8, device="cuda")
    xt, gt, bt, kt, vtt = T(x), T(gamma), T(beta), T(k), T(vt)
    qbt = None if qb is None else T(qb)
    qzt = None if qz is None else T(qz)
    qmt, qst = T(qm_), T(qs_)
    iw._lib.call("iw_attention_decode_cross_lnq", xt.data_ptr(), C, gt.data_ptr(), bt.data_ptr(), lm, ls, om, os_, 13,
                 True, wf.data_ptr(), None if qbt is None else qbt.data_ptr(),
                 None if qzt is None else qzt.data_ptr(), qmt.data_ptr(), qst.data_ptr(), bias, asym, kt.data_ptr(),
                 H * Tk * D, Tk * D, D, vtt.data_ptr(), H * D * t16, D * t16, t16, out.data_ptr(), B, H, D, Tk, qm,
                 qs, f, am, as_, 16, stream())
    torch.cuda.synchronize()
    got = _unfrag(host(out), B, C)
    assert np.array_equal(got.reshape(B, 1, C), exp)


def test_attention_decode_cross_lnq_rejects(iw, gpu):
    """Unsupported shapes fail with a message and launch nothing."""
    t = torch.zeros(1 << 16, dtype=torch.int8, device="cuda")
    p = t.data_ptr()
    base = dict(heads=20, head_dim=64, k_length=1500, batch=2)

    def call(heads, head_dim, k_length, batch):
        return iw._lib.call("iw_attention_decode_cross_lnq", p, heads * head_dim, p, None, 1, 1, 1, 1, 13, False, p,
                            None, None, p, p, False, False, p, 0, 0, 64, p, 0, 0, 1504, p, batch, heads, head_dim,
                            k_length, 1, 1, 8, 1, 1, 16, stream())
    for over, what in (({"head_dim": 96}, "head_dim 64"), ({"heads": 7}, "LayerNorm hidden size"),
                       ({"k_length": 3000}, "keys"), ({"batch": 129}, "rows")):
        kw = dict(base, **over)
        with pytest.raises(RuntimeError, match=what):
            call(**kw)


def test_fused_cross_attention_does_not_change_results(iw, gpu, tiny_model):
    """The one-token step with the cross-attention's LayerNorm and query
    projection fused into the attention kernel and as separate launches: the
    same greedy tokens (replayed graphs) and the same logits step by step."""
    dims, params = tiny_model
    model = iw.Whisper_int.from_params(dims, params).cuda()
    B, steps = 5, 19
    mel = iw.synth.synthetic_mel(B, dims.n_mels, 2 * dims.n_audio_ctx, seed=9)
    prompt = np.random.default_rng(9).integers(0, dims.n_vocab, size=(B, 3)).astype(np.int64)
    runners = [iw.DecoderRunner(model.decoder, B, dims.n_audio_ctx, fuse_cross=fc) for fc in (False, True)]
    eager = [iw.DecoderRunner(model.decoder, B, dims.n_audio_ctx, use_graph=False, fuse_cross=fc)
             for fc in (False, True)]
    assert runners[1].fuse_cross and not runners[0].fuse_cross
    with torch.no_grad():
        feats = model.embed_audio(T(mel))
        toks = [host(iw.greedy_decode(model, feats, T(prompt), steps, runner=r)) for r in runners]
        logits = [host(iw.greedy_decode(model, feats, T(prompt), steps, runner=r, keep_logits=True)[1])
                  for r in eager]
    assert np.array_equal(toks[0], toks[1])
    assert np.array_equal(logits[0], logits[1])
