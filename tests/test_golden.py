"""Golden fixtures written from the reference's own scalar kernels
(tests/golden/make_golden.py): the oracle must reproduce every one of them on
the CPU, and the HIP path through the C ABI must reproduce them on the GPU.

The fixtures pin the oracle where oracle/_ref is absent (the GPU hosts, any
machine without the reference tree); the digests pin full model shapes.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from tests import gen

GOLDEN = Path(__file__).resolve().parent / "golden"
OPS = ["linear8", "linear32", "classifier", "conv1d", "layernorm32", "rsqrt", "gelu", "residual15",
       "add_requant15", "attention"]


def load_cases(name):
    z = np.load(GOLDEN / f"{name}.npz")
    n = int(z["ncases"])
    cases = [dict() for _ in range(n)]
    for key in z.files:
        if key == "ncases":
            continue
        c, field = key.split(".", 1)
        v = z[key]
        if v.dtype.kind == "U":  # "@<key>": an array stored earlier
            v = z[str(v)[1:]]
        cases[int(c[1:])][field] = v
    return cases


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _i(c, k):
    return int(c[k]) if k in c else None


# ---------------------------------------------------------------------------
# one runner per op: ``impl`` is the oracle (numpy) or the HIP ops (torch)
# ---------------------------------------------------------------------------

class OracleImpl:
    def __init__(self, oracle):
        self.o = oracle

    def run(self, op, c):
        o = self.o
        if op == "linear8":
            return o.linear8(c["x"], c["w"], c.get("bias"), c.get("wz"), c["mult"], c["shift"])
        if op == "linear32":
            return o.linear32(c["x"], c["w"], c.get("bias"), c.get("wz"), c["mult"], c["shift"])
        if op == "classifier":
            return o.classifier(c["x"], c["w"], _i(c, "mult"), _i(c, "shift"))
        if op == "conv1d":
            return o.conv1d(c["x"], c["w"], c.get("bias"), _i(c, "mult"), _i(c, "shift"),
                            _i(c, "stride"), _i(c, "padding"))
        if op == "layernorm32":
            return o.layernorm32(c["x"], c["gamma"], c.get("beta"), _i(c, "ln_m"), _i(c, "ln_s"),
                                 _i(c, "out_m"), _i(c, "out_s"))
        if op == "rsqrt":
            return o.rsqrt(c["x"], _i(c, "offset"))
        if op == "gelu":
            return o.gelu(c["x"], c["lut"], c["luti_m"], c["luti_s"], c["luto_m"], c["luto_s"])
        if op == "residual15":
            return o.residual15(c["branch"], c["residual"], _i(c, "mult"))
        if op == "add_requant15":
            return o.add_requant15(c["x"], c["addend"], c["mult"], c["shift"])
        if op == "attention":
            qk, rm = o.qk_requant_rowmax(c["q"], c["k"], c.get("mask"), _i(c, "qk_m"), _i(c, "qk_s"))
            p, rs = o.shift_exp(qk, rm, c.get("mask"), _i(c, "frac_bits"))
            out = o.pv_norm_requant(p, c["v"], rs, _i(c, "av_m"), _i(c, "av_s"), _i(c, "rsqrt_offset"))
            return {"qk": qk, "rmp1": rm, "p": p, "row_sum": rs, "out": out}
        raise KeyError(op)


class HipImpl:
    def __init__(self, iw):
        self.k = iw.kernels

    @staticmethod
    def T(a):
        return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()

    @staticmethod
    def S(v, dtype):
        return torch.tensor([v], dtype=dtype)

    def run(self, op, c):
        k, T, S = self.k, self.T, self.S
        if op in ("linear8", "linear32"):
            fn = k.linear8_hip if op == "linear8" else k.linear32_hip
            return fn(T(c["x"]), T(c["w"]), T(c.get("bias")), T(c.get("wz")), T(c["mult"]),
                      T(c["shift"])).cpu().numpy()
        if op == "classifier":
            return k.classifier_hip(T(c["x"]), T(c["w"]), S(_i(c, "mult"), torch.uint32),
                                    S(_i(c, "shift"), torch.int8)).cpu().numpy()
        if op == "conv1d":
            return k.conv1d_hip(T(c["x"]), T(c["w"]), T(c.get("bias")), S(_i(c, "mult"), torch.uint32),
                                S(_i(c, "shift"), torch.int8), _i(c, "stride"),
                                _i(c, "padding")).cpu().numpy()
        if op == "layernorm32":
            return k.layernorm32_hip(T(c["x"]), T(c["gamma"]), T(c.get("beta")),
                                     S(_i(c, "ln_m"), torch.uint8), S(_i(c, "ln_s"), torch.int8),
                                     S(_i(c, "out_m"), torch.uint32),
                                     S(_i(c, "out_s"), torch.int8)).cpu().numpy()
        if op == "rsqrt":
            return k.layernorm32_rsqrt_hip(T(c["x"]), _i(c, "offset")).cpu().numpy()
        if op == "gelu":
            return k.gelu_hip(T(c["x"]), T(c["lut"]), T(c["luti_m"]), T(c["luti_s"]), T(c["luto_m"]),
                              T(c["luto_s"])).cpu().numpy()
        if op == "residual15":
            return k.residual15_hip(T(c["branch"]), T(c["residual"]),
                                    S(_i(c, "mult"), torch.uint16)).cpu().numpy()
        if op == "add_requant15":
            return k.add_requant15_hip(T(c["x"]), T(c["addend"]), T(c["mult"]),
                                       T(c["shift"])).cpu().numpy()
        if op == "attention":
            mask = T(c.get("mask"))
            qk, rm = k.qk_requant_rowmax_hip(T(c["q"]), T(c["k"]), mask, S(_i(c, "qk_m"), torch.uint8),
                                             S(_i(c, "qk_s"), torch.int8))
            p, rs = k.shift_exp_hip(qk, rm, mask, S(_i(c, "frac_bits"), torch.int32))
            out = k.pv_norm_requant_hip(p, T(c["v"]), rs, S(_i(c, "av_m"), torch.uint8),
                                        S(_i(c, "av_s"), torch.int8), _i(c, "rsqrt_offset"))
            return {"qk": qk.cpu().numpy(), "rmp1": rm.cpu().numpy(), "p": p.cpu().numpy(),
                    "row_sum": rs.cpu().numpy(), "out": out.cpu().numpy()}
        raise KeyError(op)


def check_op(impl, op):
    cases = load_cases(op)
    assert cases, op
    for i, c in enumerate(cases):
        got = impl.run(op, c)
        if isinstance(got, dict):
            for f, v in got.items():
                exp = c[f]
                assert np.array_equal(v.reshape(exp.shape), exp), f"{op} case {i} field {f}"
        else:
            exp = c["out"]
            assert got.dtype == exp.dtype, f"{op} case {i} dtype"
            assert np.array_equal(got.reshape(exp.shape), exp), f"{op} case {i}"


def digest_cases():
    with open(GOLDEN / "digests.json") as f:
        return json.load(f)


def digest_inputs(name, spec):
    kind = name.split(".")[0]
    if kind in ("linear8", "linear32"):
        M, K, N = spec["shape"]
        x, w, b, z, m, s = gen.realistic_linear_case(spec["seed"], M, K, N)
        if kind == "linear32":
            s[:] = np.arange(N) % spec["shift_mod"]
        return kind, (x, w, b, z, m, s)
    if kind == "layernorm32":
        return kind, gen.ln_case(spec["seed"], spec["rows"], spec["hidden"], spec["spread"])
    if kind == "attention":
        return kind, gen.attn_case(spec["seed"], *spec["shape"])
    raise KeyError(name)


def check_digests(impl):
    for name, spec in digest_cases().items():
        kind, args = digest_inputs(name, spec)
        if kind in ("linear8", "linear32"):
            got = impl.run(kind, dict(zip(("x", "w", "bias", "wz", "mult", "shift"), args)))
        elif kind == "layernorm32":
            x, g, b, lm, ls, om, os_ = args
            got = impl.run(kind, {"x": x, "gamma": g, "beta": b, "ln_m": lm, "ln_s": ls, "out_m": om,
                                  "out_s": os_})
        else:
            q, k, v, qm, qs, f, am, as_ = args
            got = impl.run(kind, {"q": q, "k": k, "v": v, "qk_m": qm, "qk_s": qs, "frac_bits": f,
                                  "av_m": am, "av_s": as_, "rsqrt_offset": 16})["out"]
        assert sha(got) == spec["sha256"], name


def model_fixture(iw):
    z = np.load(GOLDEN / "model_tiny.npz")
    dims = iw.ModelDimensions(*[int(v) for v in z["dims"]])
    params = {k[len("param."):]: z[k] for k in z.files if k.startswith("param.")}
    return dims, params, z


# ---------------------------------------------------------------------------
# CPU: the oracle against the fixtures
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("op", OPS)
def test_oracle_matches_golden(oracle, op):
    check_op(OracleImpl(oracle), op)


def test_oracle_matches_digests(oracle):
    check_digests(OracleImpl(oracle))


def test_oracle_model_matches_golden(iw):
    from oracle.model_oracle import OracleWhisper

    dims, params, z = model_fixture(iw)
    o = OracleWhisper(dims, params, threads=4)
    feats = o.encoder(z["mel_int8"])
    assert np.array_equal(feats, z["encoder_out"])
    toks, logits = o.greedy(feats, z["prompt"], z["logits"].shape[1], return_logits=True)
    assert np.array_equal(logits, z["logits"])
    assert np.array_equal(toks, z["tokens"])
    f_argmax, f_logits = o.forced(feats, z["prompt"], z["forced"])
    assert np.array_equal(f_logits, z["forced_logits"])
    assert np.array_equal(f_argmax, z["forced_argmax"])


def test_model_fixture_exercises_token_ids(iw):
    """Each row has its own prompt, and the teacher-forced steps' argmax ids vary."""
    dims, params, z = model_fixture(iw)
    assert not np.array_equal(z["prompt"][0], z["prompt"][1])
    assert all(len(np.unique(r)) >= 6 for r in z["forced_argmax"])
    assert z["forced_argmax"].max() >= 0 and z["forced_argmax"].max() < dims.n_vocab


def test_golden_fixtures_are_not_degenerate():
    """The fixtures exercise the requant paths rather than saturating everywhere."""
    lin = load_cases("linear8")
    assert sum(len(np.unique(c["out"])) > 20 for c in lin) >= 8
    att = load_cases("attention")
    assert any(int(c["p"].max()) == 128 for c in att)  # the int16 row-max wrap corner
    assert sum(len(np.unique(c["out"])) > 10 for c in att) >= 5
    ln = load_cases("layernorm32")
    assert sum(len(np.unique(c["out"])) > 50 for c in ln) >= 10


# ---------------------------------------------------------------------------
# GPU: the HIP path against the same fixtures
# ---------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("op", OPS)
def test_hip_matches_golden(iw, gpu, op):
    print("golden op:", op, flush=True)
    check_op(HipImpl(iw), op)


@pytest.mark.gpu
def test_hip_matches_digests(iw, gpu):
    check_digests(HipImpl(iw))


@pytest.mark.gpu
def test_hip_model_matches_golden(iw, gpu):
    dims, params, z = model_fixture(iw)
    model = iw.Whisper_int.from_params(dims, params).cuda()
    with torch.no_grad():
        feats = model.embed_audio(torch.from_numpy(z["mel_int8"]).cuda())
        toks, logits = iw.greedy_decode(model, feats, torch.from_numpy(z["prompt"]).cuda(),
                                        z["logits"].shape[1], keep_logits=True)
    assert np.array_equal(feats.cpu().numpy(), z["encoder_out"])
    assert np.array_equal(logits.cpu().numpy(), z["logits"])
    assert np.array_equal(toks.cpu().numpy(), z["tokens"])
    # teacher-forced steps through the runner's one-token step
    for frag in (True, False):
        run = iw.DecoderRunner(model.decoder, 2, dims.n_audio_ctx, use_graph=False, frag=frag)
        with torch.no_grad():
            run.set_audio(feats)
            f_argmax, f_logits = run.run_forced(torch.from_numpy(z["prompt"]).cuda(),
                                                torch.from_numpy(z["forced"]).cuda())
        assert np.array_equal(f_logits.cpu().numpy(), z["forced_logits"]), frag
        assert np.array_equal(f_argmax.cpu().numpy(), z["forced_argmax"]), frag
