"""Logit filters of the decoding task (decoding.py:410-509) and the greedy
update (:275-296): the CPU restatement in oracle/logit_filters.py pinned by
hand-derived answers and rule invariants, and the device-side filtered greedy
step (iw_greedy_advance_filtered) against it on the GPU."""
import numpy as np
import pytest
import torch

from oracle.logit_filters import (FilterSpec, apply_filters, greedy_next, greedy_update, timestamp_margin,
                                  token_prob)

# toy vocabulary: text 0..5, EOT 6, <|notimestamps|> 7, timestamps 8..11
TOY = FilterSpec(sample_begin=2, eot=6, suppress_tokens=[1], blank_ids=[0, 6], timestamp_begin=8,
                 no_timestamps=7, max_initial_timestamp_index=2)
TOY_LOGITS = np.array([5, 9, 1, 2, 3, 0, 4, 8, 1, 2, 3, 7], np.float32)


def toy(seq, logits=TOY_LOGITS, spec=TOY):
    return int(greedy_next(logits[None], np.array([[50, 51] + list(seq)]), spec)[0])


def test_known_answers():
    # first step: only timestamps 8..10 (max_initial 2), SuppressBlank irrelevant -> 10
    assert toy([]) == 10
    # after [ts]: penultimate counts as timestamp -> no timestamp; 1 suppressed, 7 notimestamps ->
    # max over {0:5, 2:1, 3:2, 4:3, 5:0, 6:4} = 0
    assert toy([9]) == 0
    # after [text, ts]: text < EOT masked, timestamps >= 9 allowed (pair may close at 9):
    # {6:4, 9:2, 10:3, 11:7} -> lse over {2,3,7} = 7.05 > 4 -> text masked -> 11
    assert toy([3, 9]) == 11
    # after [ts, ts]: must be text; timestamps >= 10 anyway masked -> 0
    assert toy([8, 9]) == 0
    # after [ts 10, text]: timestamps must be >= 11: {0:5 ... 6:4, 11:7}: lse_ts = 7 > 5 -> 11
    assert toy([10, 3]) == 11
    # same with a low last timestamp logit: text wins, the best text is index 0
    low = TOY_LOGITS.copy()
    low[11] = 1
    assert toy([10, 3], low) == 0
    # EOT freeze: a row whose last token is EOT keeps EOT whatever the logits
    assert toy([3, 6]) == 6
    # SuppressBlank without timestamp rules: at the first step 0 and 6 are out, later only 1
    plain = FilterSpec(sample_begin=2, eot=6, suppress_tokens=[1], blank_ids=[0, 6])
    flat = TOY_LOGITS.copy()
    flat[7] = 2
    flat[11] = 1
    assert toy([], flat, plain) == 4
    assert toy([2], flat, plain) == 0
    # everything suppressed -> 0 (argmax over -inf)
    allsup = FilterSpec(sample_begin=2, eot=6, suppress_tokens=list(range(12)))
    assert int(greedy_next(TOY_LOGITS[None], np.array([[50, 51, 2]]), allsup)[0]) == 0


def random_case(rng, B, V, tb, eot, nts_low):
    """Rows of random int8 logits with mixed timestamp ranges and histories."""
    q = rng.integers(-128, 128, size=(B, V)).astype(np.int8)
    # a part of the rows with low timestamp logits, so both outcomes of the probability rule occur
    q[:nts_low, tb:] = rng.integers(-128, -60, size=(nts_low, V - tb)).astype(np.int8)
    return q


def history_for(rng, st, V, tb, eot):
    seq = []
    for _ in range(st):
        r = rng.random()
        if r < 0.35:
            seq.append(int(rng.integers(tb, V)))
        elif r < 0.4:
            seq.append(eot)
        else:
            seq.append(int(rng.integers(0, eot)))
    return seq


def check_invariants(q, hist, spec, nxt):
    V = q.shape[1]
    tb, eot = spec.timestamp_begin, spec.eot
    for k in range(q.shape[0]):
        seq = hist[k]
        t = int(nxt[k])
        if seq and seq[-1] == eot:
            assert t == eot
            continue
        sup = set(spec.suppress_tokens) | ({spec.no_timestamps} if tb is not None else set())
        if not seq and spec.blank_ids:
            sup |= set(spec.blank_ids)
        # brute-force allowed predicate, independent of the masking code
        def ok(i):
            if i in sup:
                return False
            if tb is None:
                return True
            if not seq:
                return tb <= i <= tb + spec.max_initial_timestamp_index
            last_ts = seq[-1] >= tb
            pen_ts = len(seq) < 2 or seq[-2] >= tb
            if last_ts and pen_ts and i >= tb:
                return False
            if last_ts and not pen_ts and i < eot:
                return False
            tss = [s for s in seq if s >= tb]
            if tss and tb <= i < (tss[-1] if (last_ts and not pen_ts) else tss[-1] + 1):
                return False
            return True
        allowed = [i for i in range(V) if ok(i)]
        if not allowed:
            assert t == 0
            continue
        assert t in allowed
        # the choice is the best allowed token of its own class (text or timestamp)
        same = [i for i in allowed if (i >= tb) == (t >= tb)] if tb is not None else allowed
        best = max(q[k, i] for i in same)
        assert q[k, t] == best and t == min(i for i in same if q[k, i] == best)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_oracle_rule_invariants(seed):
    rng = np.random.default_rng(seed)
    V, tb, eot = 300, 200, 150
    spec = FilterSpec(sample_begin=3, eot=eot, suppress_tokens=[5, 17, 151, 199], blank_ids=[20, eot],
                      timestamp_begin=tb, no_timestamps=160, max_initial_timestamp_index=25)
    for st in (0, 1, 2, 3, 6, 12):
        q = random_case(rng, 24, V, tb, eot, 12)
        hist = [history_for(rng, st, V, tb, eot) for _ in range(24)]
        toks = np.array([[1, 2, 3] + h for h in hist], np.int64).reshape(24, 3 + st)
        nxt = greedy_next(q.astype(np.float32) * 0.1, toks, spec)
        check_invariants(q, hist, spec, nxt)


# ---------------------------------------------------------------------------
# GPU: iw_greedy_advance_filtered against the oracle
# ---------------------------------------------------------------------------

def bitmask(ids, V):
    m = np.zeros((V + 31) // 32, np.uint32)
    for i in ids:
        m[i >> 5] |= np.uint32(1) << np.uint32(i & 31)
    return m


@pytest.mark.gpu
@pytest.mark.parametrize("rules", ["timestamps", "plain", "none"])
def test_filtered_greedy_step_matches_oracle(iw, gpu, rules):
    print("filtered greedy:", rules, flush=True)
    rng = np.random.default_rng(7)
    V, eot, tb, nots = 51865, 50257, 50364, 50363
    sup = sorted(set(rng.integers(0, eot, 90).tolist()) | {nots - 1})
    blank = [220, eot]
    scale = 0.0917
    if rules == "timestamps":
        spec = FilterSpec(sample_begin=3, eot=eot, suppress_tokens=sup, blank_ids=blank,
                          timestamp_begin=tb, no_timestamps=nots, max_initial_timestamp_index=50)
    elif rules == "plain":
        spec = FilterSpec(sample_begin=3, eot=eot, suppress_tokens=sup, blank_ids=blank)
    else:
        spec = FilterSpec(sample_begin=3, eot=eot)
    B, hist_cols = 48, 40
    dev = "cuda"
    # the device masks are exactly the spec's suppressions
    always = list(spec.suppress_tokens) + ([nots] if spec.timestamp_begin is not None else [])
    m_all = torch.from_numpy(bitmask(always, V)).to(dev) if always else None
    m_first = torch.from_numpy(bitmask(always + (blank if spec.blank_ids else []), V)).to(dev)
    prompt = np.array([[50258, 50259, 50359]] * B, np.int64)
    prompt[::7, -1] = eot  # rows whose prompt ends in EOT stay frozen from the first step
    prev0 = torch.from_numpy(prompt[:, -1].copy()).to(dev)
    for st in (0, 1, 2, 3, 7, 20):
        q = random_case(rng, B, V, tb, eot, B // 2)
        hist = [history_for(rng, st, V, tb, eot) for _ in range(B)]
        toks = np.concatenate([prompt, np.array(hist, np.int64).reshape(B, st)], 1)
        f32 = q.astype(np.float32) * np.float32(scale)
        margin = timestamp_margin(f32, toks, spec)
        keep = margin > 1e-3
        want = greedy_next(f32, toks, spec)
        h = np.zeros((B, hist_cols), np.int64)
        h[:, :st] = np.array(hist, np.int64).reshape(B, st)
        ht = torch.from_numpy(h).to(dev)
        qt = torch.from_numpy(q).to(dev)
        nxt = torch.empty(B, dtype=torch.int64, device=dev)
        step = torch.tensor([st], dtype=torch.int32, device=dev)
        pos = torch.tensor([3 + st], dtype=torch.int32, device=dev)
        slp0 = rng.normal(-5, 2, B).astype(np.float32)
        slp = torch.from_numpy(slp0.copy()).to(dev)
        cnt = torch.zeros(hist_cols, dtype=torch.int32, device=dev)
        iw._lib.call("iw_greedy_advance_filtered", qt.data_ptr(), B, V, V, nxt.data_ptr(), ht.data_ptr(),
                     hist_cols, hist_cols, step.data_ptr(), pos.data_ptr(), 1,
                     m_all.data_ptr() if m_all is not None else None,
                     m_first.data_ptr() if spec.blank_ids else None, prev0.data_ptr(),
                     eot, spec.timestamp_begin if spec.timestamp_begin is not None else -1,
                     spec.max_initial_timestamp_index if spec.max_initial_timestamp_index is not None else -1,
                     scale, slp.data_ptr(), cnt.data_ptr(), torch.cuda.current_stream().cuda_stream)
        got = nxt.cpu().numpy()
        assert np.array_equal(got[keep], want[keep]), (st, np.nonzero(got != want))
        assert np.array_equal(ht.cpu().numpy()[:, st], got)
        assert int(step.item()) == st + 1 and int(pos.item()) == 4 + st
        assert keep.mean() > 0.9
        # GreedyDecoder.update's log-probability sum and the EOT count
        w_next, w_slp, _ = greedy_update(apply_filters(f32, toks, spec), toks, eot, slp0)
        assert np.array_equal(w_next[keep], got[keep])
        g_slp = slp.cpu().numpy()
        assert np.array_equal(np.isnan(g_slp[keep]), np.isnan(w_slp[keep]))
        fin = keep & ~np.isnan(w_slp)
        assert np.allclose(g_slp[fin], w_slp[fin], rtol=1e-5, atol=1e-4), (st, g_slp - w_slp)
        c = cnt.cpu().numpy()
        assert c[st] == int((got == eot).sum()) and c.sum() == c[st]


@pytest.mark.gpu
def test_greedy_decode_with_filters(iw, gpu):
    """End to end on the golden 1+1-layer model: every step's token is the
    filtered greedy choice over that step's int8 logits and the tokens so far,
    and the graph-replayed decode gives the same tokens as the eager one."""
    from tests.test_golden import model_fixture

    dims, params, z = model_fixture(iw)
    model = iw.Whisper_int.from_params(dims, params).cuda()
    eot, tb = 900, 905
    sup = [1, 5, 77, 901]
    filt = iw.LogitFilters(eot=eot, suppress_tokens=sup, suppress_blank=[220, eot], timestamp_begin=tb,
                           no_timestamps=904, max_initial_timestamp_index=40)
    spec = FilterSpec(sample_begin=3, eot=eot, suppress_tokens=sup, blank_ids=[220, eot], timestamp_begin=tb,
                      no_timestamps=904, max_initial_timestamp_index=40)
    steps = 12
    with torch.no_grad():
        feats = model.embed_audio(torch.from_numpy(z["mel_int8"]).cuda())
        prompt = torch.from_numpy(z["prompt"]).cuda()
        toks, logits = iw.greedy_decode(model, feats, prompt, steps, keep_logits=True, filters=filt)
        toks2 = iw.greedy_decode(model, feats, prompt, steps, filters=filt)
    toks, logits = toks.cpu().numpy(), logits.cpu().numpy()
    assert np.array_equal(toks, toks2.cpu().numpy())
    scale = np.float32(1.0 / float(params["decoder.act_logits_alpha"][0]))
    for j in range(steps):
        f32 = logits[:, j].astype(np.float32) * scale
        ctx = toks[:, :3 + j]
        keep = timestamp_margin(f32, ctx, spec) > 1e-3
        want = greedy_next(f32, ctx, spec)
        assert np.array_equal(toks[keep, 3 + j], want[keep]), j
    # the first sampled token obeys the initial-timestamp rule
    assert ((toks[:, 3] >= tb) & (toks[:, 3] <= tb + 40)).all()


def test_greedy_update_oracle_known_answers():
    """GreedyDecoder.update's bookkeeping restated (decoding.py:279-296): the
    log-probability of the argmax for uniform logits is -log(V), for two tied
    maxima -log(2) (first index chosen), agrees with torch.log_softmax on random
    rows, is not added after EOT, and the rows after EOT emit EOT."""
    V, eot = 1000, 7
    logits = np.zeros((4, V), np.float32)
    logits[1, [3, 900]] = 50.0                      # two tied maxima, far above the rest
    logits[2] = np.random.default_rng(1).normal(0, 3, V).astype(np.float32)
    logits[3, eot] = 9.0
    tokens = np.array([[1, 2], [1, 2], [1, 2], [1, eot]], np.int64)
    nxt, slp, done = greedy_update(logits, tokens, eot, np.zeros(4, np.float32))
    assert nxt.tolist()[:3] == [0, 3, int(np.argmax(logits[2]))] and nxt[3] == eot
    assert np.isclose(slp[0], -np.log(V), atol=1e-5)
    assert np.isclose(slp[1], -np.log(2), atol=1e-5)
    want2 = torch.log_softmax(torch.from_numpy(logits[2]), -1)[nxt[2]].item()
    assert np.isclose(slp[2], want2, atol=1e-5)
    assert slp[3] == 0.0 and not done
    _, _, done = greedy_update(logits[3:], tokens[3:], eot, np.zeros(1, np.float32))
    assert done
    # no-speech probability: softmax at a token
    p = token_prob(logits, 3)
    assert np.isclose(p[0], 1.0 / V) and np.isclose(p[1], 0.5, atol=1e-6)
    assert np.isclose(p[2], torch.softmax(torch.from_numpy(logits[2]), -1)[3].item(), rtol=1e-5)
