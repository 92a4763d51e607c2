"""Model-level parity at the benchmark workloads' shapes.

Each workload's model runs on the GPU at its full batch (and, with a decoder,
its full number of greedy steps) through the batched runners the benchmark
uses: EncoderRunner, then DecoderRunner replaying HIP graphs. Rows of the batch
are checked bit-exactly against the oracle (oracle/model_oracle.py, the
reference dataflow of model_int.py:1215-1622 and decoding.py:684-712 composed
from the restated scalar kernels):

* the int8 encoder output (for Whisper-base, every layer's int16 residual
  stream too);
* the int8 logits of every greedy step: the oracle runs the decoder once over
  the whole GPU token sequence (causal mask, no cache), whose position t equals
  the cached step that fed token t, and the first-index argmax of each step's
  logits must be the token the GPU chose next.

The synthetic checkpoints decode varied token streams (synth.py's shaped
decoder), so the self-attention caches hold a different token at every
position; every checked row must emit at least 8 distinct ids. The replayed
graphs' tokens equal an eager decode's, whose logits are the ones checked, and
the graphs' last-step logits equal the eager last step's.

Whisper-base runs its full 6-layer encoder. Whisper-small, -medium and -large
keep their real width, heads, mel bins, vocabulary, audio length, batch and step
count with 2 encoder + 2 decoder layers, so the oracle finishes in seconds.
Whisper-small, -medium and -large also run at full depth (12 + 12, 24 + 24 and
32 + 32 layers, medium after its seeded random prompt ids): there rows of the
full batch equal batch-1 runs of the same input at every step's int8 logits
(the kernels have no cross-row arithmetic), and rows are checked against the
oracle at full depth.
"""
import os
import time

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

# workload -> (shape, batch, greedy steps, prompt seed or None, layers or None = full)
WORKLOADS = {
    "base": ("base", 16, 0, None, None),
    "small": ("small", 32, 128, None, 2),
    "medium": ("medium", 64, 224, 4, 2),
    "large": ("large", 128, 445, None, 2),
}
MIN_DISTINCT = 8


def _threads():
    return max(1, min(16, os.cpu_count() or 1))


def _dims(iw, shape, layers):
    d = iw.SHAPES[shape]
    if layers is None:
        return d
    return iw.ModelDimensions(d.n_mels, d.n_audio_ctx, d.n_audio_state, d.n_audio_head, layers, d.n_vocab,
                              d.n_text_ctx, d.n_text_state, d.n_text_head, layers)


def _log(*a):
    print(*a, flush=True)


def oracle_check(dims, params, mel, prompt, feats, tokens, logits, layer_streams=None, kind="oracle"):
    """Bit-exact oracle check of one or more rows: ``mel`` float32 [R, n_mels, F];
    GPU results for the same rows: ``feats`` int8 encoder output, ``tokens``
    [R, P + steps] (or None), ``logits`` int8 [R, steps, vocab] (or None),
    ``layer_streams`` list of int16 residual streams after each encoder block."""
    from oracle.model_oracle import OracleWhisper

    ref = OracleWhisper(dims, params, threads=_threads(), kind=kind)
    t0 = time.time()
    if layer_streams is not None:
        x = ref.encoder_frontend(mel)
        for i, got in enumerate(layer_streams):
            x = ref._block(x, None, None, None, f"encoder.blocks.{i}", dims.n_audio_head, False)
            assert np.array_equal(got, x), f"encoder block {i}"
        xa = ref._ln(x, "encoder.ln_post")
    else:
        xa = ref.encoder(mel)
    assert np.array_equal(feats, xa), "encoder output"
    _log(f"  oracle encoder {time.time() - t0:.1f} s")
    if tokens is None:
        return
    P = prompt.shape[1]
    assert np.array_equal(tokens[:, :P], prompt)
    t0 = time.time()
    # position t of one causal pass over tokens[:, :-1] = the cached step that fed token t
    full = ref.decoder_logits(np.ascontiguousarray(tokens[:, :-1]), xa)
    step_logits = full[:, P - 1:]
    if logits is not None:
        assert np.array_equal(logits, step_logits), "int8 logits"
    assert np.array_equal(np.argmax(step_logits, -1), tokens[:, P:]), "greedy tokens"
    _log(f"  oracle decoder {time.time() - t0:.1f} s")


def _varied(tokens, P):
    for r, row in enumerate(tokens):
        n = len(set(row[P:].tolist()))
        assert n >= MIN_DISTINCT, f"row {r} emits only {n} distinct ids"


def _decode_both(iw, model, feats, prompt, steps, B, n_audio_ctx):
    """Graph-replayed decode (tokens) and eager decode (tokens and every step's
    logits); the two token streams and the last step's logits must agree."""
    dec = iw.DecoderRunner(model.decoder, B, n_audio_ctx)
    tg = iw.greedy_decode(model, feats, prompt, steps, runner=dec)
    last = dec.logits.clone()
    te, lg = iw.greedy_decode(model, feats, prompt, steps, keep_logits=True)
    torch.cuda.synchronize()
    assert torch.equal(tg, te), "graph-replayed and eager decoding differ"
    assert torch.equal(last, lg[:, -1]), "graph-replayed last-step logits differ from eager"
    del dec
    return tg, lg


@pytest.mark.parametrize("name", list(WORKLOADS))
def test_workload_rows_match_oracle(iw, gpu, name):
    shape, B, steps, pseed, layers = WORKLOADS[name]
    dims = _dims(iw, shape, layers)
    _log(f"workload {name}: batch {B}, {steps} steps, layers {dims.n_audio_layer}+{dims.n_text_layer}")
    params = iw.synth.calibrated_int_params(dims, seed=100 + B)
    model = iw.Whisper_int.from_params(dims, params).cuda().eval()
    mel = iw.synth.synthetic_mel(B, dims.n_mels, 2 * dims.n_audio_ctx, seed=200 + B)
    rows = [0, B - 1]
    enc = iw.EncoderRunner(model.encoder, B)
    streams = None
    with torch.no_grad():
        if steps == 0:
            # every layer's residual stream of the two rows
            x16 = model.encoder.frontend(torch.from_numpy(mel).cuda())
            streams = []
            for i in range(dims.n_audio_layer):
                enc.block(i, x16)
                streams.append(x16.view(B, dims.n_audio_ctx, -1)[rows].cpu().numpy())
            feats = enc(torch.from_numpy(mel).cuda())
        else:
            feats = enc(torch.from_numpy(mel).cuda())
    torch.cuda.synchronize()
    tokens = logits = prompt = None
    if steps:
        prompt = iw.synth.prompt_tokens(B, dims.n_vocab, seed=pseed)
        with torch.no_grad():
            tg, lg = _decode_both(iw, model, feats, torch.from_numpy(prompt).cuda(), steps, B, dims.n_audio_ctx)
        tokens = tg[rows].cpu().numpy()
        logits = lg[rows].cpu().numpy()
        assert tokens.min() >= 0 and tokens.max() < dims.n_vocab
        del lg
        _log(f"  gpu tokens row 0: {tokens[0, :12].tolist()} ...")
        _varied(tokens, prompt.shape[1])
    oracle_check(dims, params, mel[rows], None if prompt is None else prompt[rows],
                 feats[rows].cpu().numpy(), tokens, logits, streams)


# shape -> (batch, greedy steps, prompt seed or None, rows checked against batch-1 runs, rows
# checked against the oracle)
FULL_DEPTH = {
    "small": (32, 128, None, (0, 31), (0, 31)),
    "medium": (64, 224, 4, (0, 41, 63), (41,)),
    "large": (128, 445, None, (0, 77, 127), (77,)),
}


@pytest.mark.parametrize("shape", list(FULL_DEPTH))
def test_full_depth(iw, gpu, shape):
    """Full depth at the workload's batch and step count: the encoder and every
    step's int8 logits of the listed rows equal batch-1 runs of the same mels,
    and the oracle rows match at full depth (encoder output, the logits of every
    step, the greedy tokens)."""
    dims = iw.SHAPES[shape]
    B, steps, pseed, batch1_rows, oracle_rows = FULL_DEPTH[shape]
    _log(f"full depth {shape}: {dims.n_audio_layer}+{dims.n_text_layer} layers, batch {B}, {steps} steps")
    t0 = time.time()
    params = iw.synth.calibrated_int_params(dims, seed=0)
    _log(f"  checkpoint {time.time() - t0:.1f} s")
    model = iw.Whisper_int.from_params(dims, params).cuda().eval()
    mel = iw.synth.synthetic_mel(B, dims.n_mels, 2 * dims.n_audio_ctx, seed=1)
    prompt = torch.from_numpy(iw.synth.prompt_tokens(B, dims.n_vocab, seed=pseed)).cuda()
    with torch.no_grad():
        feats = iw.EncoderRunner(model.encoder, B)(torch.from_numpy(mel).cuda()).clone()
        toks, lg = _decode_both(iw, model, feats, prompt, steps, B, dims.n_audio_ctx)
        assert int(toks.min()) >= 0 and int(toks.max()) < dims.n_vocab
        rows = sorted(set(batch1_rows) | set(oracle_rows))
        keep = {r: (feats[r].cpu().numpy(), toks[r].cpu().numpy(), lg[r].cpu().numpy()) for r in rows}
        del lg
        _log(f"  batch {B} done; row 0 tokens {keep[rows[0]][1][3:15].tolist()} ...")
        _varied(np.stack([keep[r][1] for r in rows]), 3)
        for r in batch1_rows:
            f1 = iw.EncoderRunner(model.encoder, 1)(torch.from_numpy(mel[r:r + 1]).cuda())
            assert np.array_equal(f1[0].cpu().numpy(), keep[r][0]), f"encoder row {r}"
            t1, l1 = iw.greedy_decode(model, f1, prompt[r:r + 1], steps, keep_logits=True)
            assert np.array_equal(l1[0].cpu().numpy(), keep[r][2]), f"int8 logits row {r}"
            assert np.array_equal(t1[0].cpu().numpy(), keep[r][1]), f"tokens row {r}"
            _log(f"  row {r}: batch-1 run equal at every step")
    del model
    torch.cuda.empty_cache()
    for r in oracle_rows:
        f, t, l = keep[r]
        oracle_check(dims, params, mel[r:r + 1], prompt[r:r + 1].cpu().numpy(), f[None], t[None], l[None],
                     kind="simd")
        _log(f"  row {r}: oracle equal at full depth")


def _straddle(params, prefix):
    """Rewrite the Linear requant parameters under ``prefix`` to an equivalent
    form whose multipliers straddle 2^31: in every other 256-column tile, every
    third channel takes m * 2 with the shift moved by one (right shifts + 1 for
    Linear8, left shifts - 1 for Linear32), so some tiles mix multipliers on both
    sides of 2^31 and the rest stay below it."""
    P = dict(params)
    n_changed = 0
    for k in [k for k in params if k.startswith(prefix) and k.endswith(".req_multiplier")]:
        base = k[: -len(".req_multiplier")]
        m = params[k].astype(np.uint64).copy()
        s = params[base + ".req_shiftmount"].astype(np.int64).copy()
        if m.size < 2:
            continue
        out_linear = base.endswith(".out") or base.endswith(".mlp.2")
        n = np.arange(m.size)
        pick = ((n // 256) % 2 == 1) & (n % 3 == 0)
        pick &= (s >= 1) if out_linear else (s <= 31)
        m[pick] *= 2
        s[pick] += -1 if out_linear else 1
        P[k] = m.astype(np.uint32)
        P[base + ".req_shiftmount"] = s.astype(np.int8)
        n_changed += int(pick.sum())
    assert n_changed > 0
    return P


def test_multipliers_straddling_2_31(iw, gpu):
    """Whisper-large shapes (2 + 2 layers, batch 8, 24 steps) with the first
    encoder and decoder blocks' Linear multipliers straddling 2^31 (reference
    checkpoints hold [2^30, 2^31]; the kernels take any uint32)."""
    dims = _dims(iw, "large", 2)
    B, steps = 8, 24
    base = iw.synth.calibrated_int_params(dims, seed=55, calib_tokens=32)
    params = _straddle(_straddle(base, "encoder.blocks.0."), "decoder.blocks.0.")
    mults = np.concatenate([params[k].ravel() for k in params
                            if k.startswith("encoder.blocks.0.") and k.endswith("req_multiplier")
                            and params[k].dtype == np.uint32])
    assert mults.min() < 2 ** 31 <= mults.max()
    model = iw.Whisper_int.from_params(dims, params).cuda().eval()
    mel = iw.synth.synthetic_mel(B, dims.n_mels, 2 * dims.n_audio_ctx, seed=56)
    prompt = iw.synth.prompt_tokens(B, dims.n_vocab, seed=57)
    with torch.no_grad():
        feats = iw.EncoderRunner(model.encoder, B)(torch.from_numpy(mel).cuda())
        tg, lg = _decode_both(iw, model, feats, torch.from_numpy(prompt).cuda(), steps, B, dims.n_audio_ctx)
    rows = [0, B - 1]
    oracle_check(dims, params, mel[rows], prompt[rows], feats[rows].cpu().numpy(), tg[rows].cpu().numpy(),
                 lg[rows].cpu().numpy())
