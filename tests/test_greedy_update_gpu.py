"""The greedy step's bookkeeping on the device (GreedyDecoder.update,
decoding.py:280-296; DecodingTask._main_loop, :684-712):

* the classifier with the argmax fused into its epilogue writes the int8
  logits and, per 32-column tile, each row's first maximum;
* iw_greedy_update turns those tile maxima (or the logits) into the first-index
  argmax, applies the EOT freeze, adds the log-probability of the token to the
  row's sum (not after EOT), counts the rows at EOT and advances the counters;
* iw_token_prob gives the no-speech probability;

against the oracle restatement in oracle/logit_filters.py, and end to end
through DecoderRunner on the golden 1+1-layer model.
"""
import numpy as np
import pytest
import torch

from oracle.logit_filters import greedy_update, token_prob
from tests import gen
from tests.test_frag_gpu import host, pack, stream

pytestmark = pytest.mark.gpu


def tile_maxima(logits):
    """[R, N] int8 -> [R, ceil(N / 32)] uint16: (y + 128) << 5 | (31 - first column of the max)."""
    R, N = logits.shape
    tiles = (N + 31) // 32
    pad = np.full((R, tiles * 32), -128, np.int32)
    pad[:, :N] = logits
    t = pad.reshape(R, tiles, 32)
    col = t.argmax(-1)
    val = t.max(-1)
    return (((val + 128) << 5) | (31 - col)).astype(np.uint16)


# (128, 1280, 51865), (1, 384, 51865), (77, 768, 20000), (33, 1280, 51865) and (100, 1024, 17000) take
# the streaming kernel (at least two column tiles per CU; Kp = 640, 960 and 1280, partial m-subtiles)
@pytest.mark.parametrize("M,K,N", [(128, 1280, 51865), (3, 512, 1000), (1, 384, 51865), (40, 768, 70),
                                   (77, 768, 20000), (33, 1280, 51865), (100, 1024, 17000)])
def test_classifier_argmax_frag(iw, oracle, gpu, M, K, N):
    print("case: classifier_argmax_frag", M, K, N, flush=True)
    r = gen.rng(M + K + N + 1)
    x = gen.i8(r, (M, K))
    w = gen.i8(r, (N, K))
    xf, wf = pack(iw, x), pack(iw, w)
    tiles = (N + 31) // 32
    for mult, shift in ((int(r.integers(2**28, 2**32)), 12), (0x80000000, 40), (777, 0)):
        want = oracle.classifier(x[None], w, mult, shift)[0]
        out = torch.empty((M, N), dtype=torch.int8, device="cuda")
        # the tile maxima with a guard region after them, which must stay untouched
        guarded = torch.full((M * tiles + 64,), 0x5A5A, dtype=torch.int16, device="cuda")
        rm = guarded[:M * tiles].view(M, tiles)
        iw._lib.call("iw_classifier_argmax_frag", xf.data_ptr(), wf.data_ptr(), mult, shift, out.data_ptr(),
                     rm.data_ptr(), M, K, N, stream())
        rm2 = torch.zeros((M, tiles), dtype=torch.int16, device="cuda")
        iw._lib.call("iw_classifier_argmax_frag", xf.data_ptr(), wf.data_ptr(), mult, shift, None,
                     rm2.data_ptr(), M, K, N, stream())
        torch.cuda.synchronize()
        assert np.array_equal(host(out), want)
        assert np.array_equal(host(rm).view(np.uint16), tile_maxima(want))
        assert torch.equal(rm, rm2)
        assert bool((guarded[M * tiles:] == 0x5A5A).all())


def _planted_logits(rng, B, V, eot, step):
    """Random int8 logits with planted rows: the maximum at EOT, tied maxima
    (first index must win), and a row saturated at 127 everywhere."""
    q = rng.integers(-127, 100, size=(B, V)).astype(np.int8)
    q[step % B, eot] = 127
    i, j = sorted(rng.choice(V, 2, replace=False))
    q[(step + 1) % B, [i, j]] = 126
    q[(step + 2) % B] = 127
    return q


@pytest.mark.parametrize("from_tiles", [True, False])
def test_greedy_update_matches_oracle(iw, gpu, from_tiles):
    rng = np.random.default_rng(11 + from_tiles)
    B, V, eot, S, P, hist_cols = 12, 51865, 50257, 9, 3, 16
    scale = 0.0731
    dev = "cuda"
    prompt = rng.integers(0, V, size=(B, P)).astype(np.int64)
    prompt[5, -1] = eot  # frozen from the first step
    prev0 = torch.from_numpy(prompt[:, -1].copy()).to(dev)
    hist = torch.zeros((B, hist_cols), dtype=torch.int64, device=dev)
    nxt = torch.empty(B, dtype=torch.int64, device=dev)
    step = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    slp = torch.zeros(B, dtype=torch.float32, device=dev)
    cnt = torch.zeros(hist_cols, dtype=torch.int32, device=dev)
    arrive = torch.zeros(1, dtype=torch.int32, device=dev)
    tokens = prompt.copy()
    w_slp = np.zeros(B, np.float32)
    tiles = (V + 31) // 32
    for st in range(S):
        q = _planted_logits(rng, B, V, eot, st)
        qt = torch.from_numpy(q).to(dev)
        rm = torch.from_numpy(tile_maxima(q).view(np.int16)).to(dev) if from_tiles else None
        iw._lib.call("iw_greedy_update", rm.data_ptr() if from_tiles else None, tiles, qt.data_ptr(), V, B, V,
                     nxt.data_ptr(), hist.data_ptr(), hist_cols, hist_cols, step.data_ptr(), pos.data_ptr(),
                     1 if st else P, eot, prev0.data_ptr(), slp.data_ptr(), scale, cnt.data_ptr(),
                     arrive.data_ptr(), stream())
        w_next, w_slp, done = greedy_update(q.astype(np.float32) * np.float32(scale), tokens, eot, w_slp)
        tokens = np.concatenate([tokens, w_next[:, None]], 1)
        torch.cuda.synchronize()
        print(f"step {st}: tokens {host(nxt)[:6].tolist()} ...", flush=True)
        assert np.array_equal(host(nxt), w_next), st
        assert np.array_equal(host(hist)[:, st], w_next)
        assert int(step.item()) == st + 1 and int(arrive.item()) == 0
        assert int(host(cnt)[st]) == int((w_next == eot).sum())
        assert np.allclose(host(slp), w_slp, rtol=1e-5, atol=1e-4), (st, host(slp) - w_slp)
    assert int(pos.item()) == P + S - 1
    assert (tokens[:, P:] == eot).any()


def test_token_prob_matches_oracle(iw, gpu):
    rng = np.random.default_rng(5)
    B, V = 7, 51865
    q = rng.integers(-127, 128, size=(B, V)).astype(np.int8)
    q[2] = 0  # uniform row
    q[3, 50362] = 127
    for scale, token in ((0.05, 50362), (0.31, 0), (1.7, V - 1)):
        out = torch.empty(B, dtype=torch.float32, device="cuda")
        qt = torch.from_numpy(q).cuda()
        iw._lib.call("iw_token_prob", qt.data_ptr(), B, V, V, token, scale, out.data_ptr(), stream())
        want = token_prob(q.astype(np.float32) * np.float32(scale), token)
        assert np.allclose(host(out), want, rtol=2e-5, atol=1e-9), (scale, host(out), want)


def test_runner_bookkeeping_end_to_end(iw, gpu):
    """DecoderRunner with the EOT id, the no-speech id and early stopping on the
    golden 1+1-layer model, graph-replayed and eager: the tokens are the
    oracle's greedy tokens with the EOT freeze, cut at the step where every row
    is at EOT; the log-probability sums and the no-speech probabilities follow
    the oracle's int8 logits through the float32 restatement. The prompts are
    chosen so that the rows reach the token used as EOT after 2, 3 and 0 other
    tokens."""
    from oracle.model_oracle import OracleWhisper
    from tests.test_golden import model_fixture

    dims, params, z = model_fixture(iw)
    model = iw.Whisper_int.from_params(dims, params).cuda()
    ref = OracleWhisper(dims, params, threads=4)
    feats = ref.encoder(z["mel_int8"])[[0, 1, 1]]
    prompt = np.array([[383, 822, 229], [815, 670, 2], [6, 543, 772]], np.int64)
    eot, no_speech, steps = 68, 17, 20
    toks0, logits0 = ref.greedy(feats, prompt, steps, return_logits=True)
    alpha = np.float32(params["decoder.act_logits_alpha"][0])
    tokens = prompt.copy()
    w_slp = np.zeros(3, np.float32)
    w_steps = steps
    for j in range(steps):
        nxt, w_slp, done = greedy_update(logits0[:, j].astype(np.float32) / alpha, tokens, eot, w_slp)
        tokens = np.concatenate([tokens, nxt[:, None]], 1)
        if done:
            w_steps = j + 1
            break
    print("expected tokens", tokens.tolist(), "sum_logprobs", w_slp.tolist(), flush=True)
    assert w_steps == 4
    # the rows repeat EOT once there, so the unfrozen oracle run fed the same tokens
    assert np.array_equal(tokens, toks0[:, :3 + w_steps])
    w_ns = token_prob(ref.decoder_logits(prompt, feats)[:, 0].astype(np.float32) / alpha, no_speech)
    for use_graph in (True, False):
        runner = iw.DecoderRunner(model.decoder, 3, dims.n_audio_ctx, use_graph=use_graph, eot=eot,
                                  no_speech=no_speech)
        with torch.no_grad():
            res = iw.greedy_decode(model, torch.from_numpy(feats).cuda(), torch.from_numpy(prompt).cuda(), steps,
                                   runner=runner, stop_on_eot=True, return_result=True)
        assert res.steps == w_steps, use_graph
        assert np.array_equal(host(res.tokens), tokens)
        assert np.allclose(host(res.sum_logprobs), w_slp, rtol=1e-5, atol=1e-4)
        assert np.allclose(host(res.no_speech_probs), w_ns, rtol=2e-5, atol=1e-9)
    # without early stopping: the fixed number of steps, EOT repeated after the finish
    with torch.no_grad():
        res = iw.greedy_decode(model, torch.from_numpy(feats).cuda(), torch.from_numpy(prompt).cuda(), steps,
                               eot=eot, return_result=True)
    assert res.steps == steps and (host(res.tokens)[:, 3 + w_steps:] == eot).all()
    assert np.allclose(host(res.sum_logprobs), w_slp, rtol=1e-5, atol=1e-4)
