"""Model-level bit-exact parity of the gfx950 path against the end-to-end oracle.

The layer API (Whisper_int and its layers, reference-style hook KV cache) and
the batched runners are compared with oracle/model_oracle.py on seeded
synthetic mels and calibrated synthetic checkpoints: int8 encoder output,
per-layer int16 residual streams, int8 logits before dequant, dequantised
logits and greedy token ids.
"""
import numpy as np
import pytest
import torch

from tests import gen

pytestmark = pytest.mark.gpu


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def small_dims(iw, heads=6, d=384, layers=2, ctx=64, n_mels=80, vocab=512, text_ctx=32):
    return iw.ModelDimensions(n_mels=n_mels, n_audio_ctx=ctx, n_audio_state=d, n_audio_head=heads,
                              n_audio_layer=layers, n_vocab=vocab, n_text_ctx=text_ctx,
                              n_text_state=d, n_text_head=heads, n_text_layer=layers)


@pytest.fixture(scope="module")
def small(iw, gpu):
    from oracle.model_oracle import OracleWhisper

    dims = small_dims(iw)
    P = iw.synth.calibrated_int_params(dims, seed=11)
    model = iw.Whisper_int.from_params(dims, P).cuda()
    return dims, P, model, OracleWhisper(dims, P)


def test_layers_match_oracle(iw, small):
    dims, P, model, ref = small
    r = gen.rng(3)
    blk = model.encoder.blocks[0]
    x16 = r.integers(-9000, 9000, size=(2, 64, 384)).astype(np.int16)
    x8 = gen.i8(r, (2, 64, 384), -127, 127)
    p = "encoder.blocks.0"
    assert np.array_equal(host(blk.attn_ln(T(x16))[0]), ref._ln(x16, p + ".attn_ln"))
    assert np.array_equal(host(blk.attn.query(T(x8))), ref._lin8(x8, p + ".attn.query"))
    assert np.array_equal(host(blk.attn.out(T(x8))), ref._lin32(x8, p + ".attn.out"))
    h = gen.i8(r, (2, 64, 1536), -127, 127)
    assert np.array_equal(host(blk.mlp[1](T(h))), ref._gelu(h, p + ".mlp.1"))
    assert np.array_equal(host(blk.attn(T(x8))), ref._mha(x8, None, None, None, p + ".attn", 6))
    assert np.array_equal(host(blk(T(x16))), ref._block(x16, None, None, None, p, 6, False))
    mel8 = gen.i8(r, (2, 80, 128), -127, 127)
    assert np.array_equal(host(model.encoder.conv1(T(mel8))), ref._conv(mel8, "encoder.conv1", 1))


def test_encoder_layer_api(iw, small):
    dims, P, model, ref = small
    mel = iw.synth.synthetic_mel(2, dims.n_mels, 2 * dims.n_audio_ctx, seed=21)
    with torch.no_grad():
        got = host(model.embed_audio(T(mel)))
    assert np.array_equal(got, ref.encoder(mel))
    # int8 input (already quantised) takes the same path
    with torch.no_grad():
        got8 = host(model.encoder(T(ref.encoder_input(mel))))
    assert np.array_equal(got8, ref.encoder(mel))


def test_encoder_runner(iw, small):
    dims, P, model, ref = small
    mel = iw.synth.synthetic_mel(3, dims.n_mels, 2 * dims.n_audio_ctx, seed=22)
    run = iw.EncoderRunner(model.encoder, 3)
    got = host(run(T(mel)))
    assert np.array_equal(got, ref.encoder(mel))
    # second call reuses the buffers
    mel2 = iw.synth.synthetic_mel(3, dims.n_mels, 2 * dims.n_audio_ctx, seed=23)
    assert np.array_equal(host(run(T(mel2))), ref.encoder(mel2))


def test_decoder_reference_style_cache(iw, small):
    """TextDecoder_int.forward with install_kv_cache_hooks, as decoding.py drives it."""
    dims, P, model, ref = small
    mel = iw.synth.synthetic_mel(2, dims.n_mels, 2 * dims.n_audio_ctx, seed=31)
    xa = ref.encoder(mel)
    prompt = np.array([[1, 2, 3], [4, 5, 6]], np.int64)
    cache, hooks = model.install_kv_cache_hooks()
    model.decoder.dequant_need = False
    ocache = {}
    toks, otoks = T(prompt), prompt
    try:
        for step in range(5):
            inp = toks if step == 0 else toks[:, -1:]
            oinp = otoks if step == 0 else otoks[:, -1:]
            got = host(model.decoder(inp, T(xa), kv_cache=cache))
            exp = ref.decoder_logits(oinp, xa, ocache)
            assert np.array_equal(got, exp), step
            nxt = exp[:, -1].argmax(-1)
            toks = torch.cat([toks, T(nxt[:, None])], 1)
            otoks = np.concatenate([otoks, nxt[:, None]], 1)
    finally:
        for h in hooks:
            h.remove()
        model.decoder.dequant_need = True
    # dequantised logits without a cache: the whole sequence at once
    got = model.decoder(toks, T(xa))
    exp = ref.decoder_logits(otoks, xa).astype(np.float32) / np.float32(P["decoder.act_logits_alpha"][0])
    assert np.array_equal(host(got), exp)


@pytest.mark.parametrize("batch,steps", [(1, 6), (3, 10)])
def test_greedy_decode_runner(iw, small, batch, steps):
    dims, P, model, ref = small
    mel = iw.synth.synthetic_mel(batch, dims.n_mels, 2 * dims.n_audio_ctx, seed=41 + batch)
    prompt = gen.rng(batch).integers(0, dims.n_vocab, size=(batch, 3)).astype(np.int64)
    with torch.no_grad():
        feats = model.embed_audio(T(mel))
        toks, logits = iw.greedy_decode(model, feats, T(prompt), steps, keep_logits=True)
    xa = ref.encoder(mel)
    etoks, elogits = ref.greedy(xa, prompt, steps, return_logits=True)
    assert np.array_equal(host(logits), elogits)
    assert np.array_equal(host(toks), etoks)


def test_greedy_decode_row_major_step(iw, small):
    """The one-token step on row-major operands (DecoderRunner(frag=False), the
    layer kernels of the prompt step) gives the oracle's logits and tokens too."""
    dims, P, model, ref = small
    batch, steps = 2, 6
    mel = iw.synth.synthetic_mel(batch, dims.n_mels, 2 * dims.n_audio_ctx, seed=43)
    prompt = gen.rng(7).integers(0, dims.n_vocab, size=(batch, 3)).astype(np.int64)
    with torch.no_grad():
        feats = model.embed_audio(T(mel))
        runner = iw.DecoderRunner(model.decoder, batch, feats.shape[1], use_graph=False, frag=False)
        assert not runner.frag
        toks, logits = iw.greedy_decode(model, feats, T(prompt), steps, runner=runner, keep_logits=True)
    xa = ref.encoder(mel)
    etoks, elogits = ref.greedy(xa, prompt, steps, return_logits=True)
    assert np.array_equal(host(logits), elogits)
    assert np.array_equal(host(toks), etoks)


def test_head_dim_96_and_128(iw, gpu):
    """Head sizes of the tiny (4 heads of 96) and the 10-head large-like shapes."""
    from oracle.model_oracle import OracleWhisper

    for heads, d in ((4, 384), (10, 1280)):
        dims = small_dims(iw, heads=heads, d=d, layers=1, ctx=40, vocab=300, text_ctx=24)
        P = iw.synth.calibrated_int_params(dims, seed=5)
        model = iw.Whisper_int.from_params(dims, P).cuda()
        ref = OracleWhisper(dims, P)
        mel = iw.synth.synthetic_mel(2, dims.n_mels, 80, seed=6)
        with torch.no_grad():
            f = model.embed_audio(T(mel))
            toks = iw.greedy_decode(model, f, T(np.array([[7, 8, 9]] * 2)), 5)
        xa = ref.encoder(mel)
        assert np.array_equal(host(f), xa)
        assert np.array_equal(host(toks), ref.greedy(xa, np.array([[7, 8, 9]] * 2), 5))


def test_config1_tiny_full(iw, gpu):
    """Whisper-tiny shapes as the reference's CPU case: d=384, 4 heads (head_dim 96),
    4+4 layers, 1500 frames, vocab 51865, batch 1, 32 greedy steps."""
    from oracle.model_oracle import OracleWhisper

    dims = iw.ModelDimensions(80, 1500, 384, 4, 4, 51865, 448, 384, 4, 4)
    P = iw.synth.calibrated_int_params(dims, seed=2024)
    model = iw.Whisper_int.from_params(dims, P).cuda()
    ref = OracleWhisper(dims, P)
    mel = iw.synth.synthetic_mel(1, 80, 3000, seed=1)
    prompt = iw.synth.prompt_tokens(1, dims.n_vocab)
    with torch.no_grad():
        f = model.embed_audio(T(mel))
        toks, logits = iw.greedy_decode(model, f, T(prompt), 32, keep_logits=True)
    xa = ref.encoder(mel)
    assert np.array_equal(host(f), xa)
    etoks, elogits = ref.greedy(xa, prompt, 32, return_logits=True)
    assert np.array_equal(host(logits), elogits)
    assert np.array_equal(host(toks), etoks)
