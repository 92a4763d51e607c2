"""Model-level parity at the benchmark workloads' shapes.

Each workload's model runs on the GPU at its full batch (and, with a decoder,
its full number of greedy steps) through the batched runners the benchmark
uses: EncoderRunner, then DecoderRunner replaying HIP graphs. Two rows (the
first and the last of the batch) are checked bit-exactly against the oracle
(oracle/model_oracle.py, the reference dataflow of model_int.py:1215-1622 and
decoding.py:684-712 composed from the restated scalar kernels):

* the int8 encoder output (for Whisper-base, every layer's int16 residual
  stream too);
* the int8 logits of every greedy step: the oracle runs the decoder once over
  the whole GPU token sequence (causal mask, no cache), whose position t equals
  the cached step that fed token t, and the first-index argmax of each step's
  logits must be the token the GPU chose next.

Whisper-base runs its full 6-layer encoder. Whisper-small, -medium and -large
keep their real width, heads, mel bins, vocabulary, audio length, batch and step
count with 2 encoder + 2 decoder layers, so the oracle finishes in seconds.
Whisper-large also runs at its full depth (32 + 32 layers): there every row
of the batch-128 run must equal a batch-1 run of the same input (the kernels
have no cross-row arithmetic), and all tokens lie in the vocabulary.
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


def oracle_check(dims, params, mel, prompt, feats, tokens, logits, layer_streams=None):
    """Bit-exact oracle check of one or more rows: ``mel`` float32 [R, n_mels, F];
    GPU results for the same rows: ``feats`` int8 encoder output, ``tokens``
    [R, P + steps] (or None), ``logits`` int8 [R, steps, vocab] (or None),
    ``layer_streams`` list of int16 residual streams after each encoder block."""
    from oracle.model_oracle import OracleWhisper

    ref = OracleWhisper(dims, params, threads=_threads())
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
        dec = iw.DecoderRunner(model.decoder, B, dims.n_audio_ctx)
        with torch.no_grad():
            tg = iw.greedy_decode(model, feats, torch.from_numpy(prompt).cuda(), steps, runner=dec)
            te, lg = iw.greedy_decode(model, feats, torch.from_numpy(prompt).cuda(), steps, keep_logits=True)
        torch.cuda.synchronize()
        assert torch.equal(tg, te), "graph-replayed and eager decoding differ"
        tokens = tg[rows].cpu().numpy()
        logits = lg[rows].cpu().numpy()
        assert tokens.min() >= 0 and tokens.max() < dims.n_vocab
        del lg
        _log(f"  gpu tokens row 0: {tokens[0, :12].tolist()} ...")
    oracle_check(dims, params, mel[rows], None if prompt is None else prompt[rows],
                 feats[rows].cpu().numpy(), tokens, logits, streams)


def test_large_full_depth_batch_invariance(iw, gpu):
    """Whisper-large at full depth, batch 128, 445 greedy steps: rows 0, 77 and
    127 equal batch-1 runs of the same mels."""
    dims = iw.SHAPES["large"]
    B, steps = 128, 445
    params = iw.synth.calibrated_int_params(dims, seed=0)
    model = iw.Whisper_int.from_params(dims, params).cuda().eval()
    mel = iw.synth.synthetic_mel(B, dims.n_mels, 2 * dims.n_audio_ctx, seed=1)
    prompt = torch.from_numpy(iw.synth.prompt_tokens(B, dims.n_vocab)).cuda()
    with torch.no_grad():
        feats = iw.EncoderRunner(model.encoder, B)(torch.from_numpy(mel).cuda()).clone()
        toks = iw.greedy_decode(model, feats, prompt, steps, runner=iw.DecoderRunner(model.decoder, B, 1500))
        torch.cuda.synchronize()
        _log(f"batch 128 done; row 0 tokens {toks[0, :10].tolist()} ...")
        assert int(toks.min()) >= 0 and int(toks.max()) < dims.n_vocab
        for r in (0, 77, 127):
            f1 = iw.EncoderRunner(model.encoder, 1)(torch.from_numpy(mel[r:r + 1]).cuda())
            assert torch.equal(f1[0], feats[r]), f"encoder row {r}"
            t1 = iw.greedy_decode(model, f1, prompt[r:r + 1], steps,
                                  runner=iw.DecoderRunner(model.decoder, 1, 1500))
            assert torch.equal(t1[0], toks[r]), f"tokens row {r}"
            _log(f"  row {r} equal")
