"""Writes the golden fixtures in tests/golden/ from the reference's own scalar
kernels (i_whisper/kernels/csrc/*/*_scalar.cpp compiled into oracle/_ref by
``make -C oracle ref``; the build reads the sources where they lie in the
reference tree and copies nothing).

Run from the repository root, where the reference tree is present:

    make -C oracle ref && python tests/golden/make_golden.py

Each fixture file ``<op>.npz`` holds, per case ``c<i>``, the inputs and the
reference kernel's outputs (``c<i>.<name>``) plus scalar parameters. The
``digests.json`` file holds SHA-256 digests of reference outputs at full model
shapes whose inputs are regenerated from a seed by tests/gen.py (numpy PCG64
streams are stable across numpy versions), so the fixtures stay small.
``model_tiny.npz`` holds an end-to-end case: the reference kernels composed
along the reference dataflow for a 1+1-layer model.

The fixtures are data: inputs and the outputs the reference produced for them.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle.oracle import Oracle, available  # noqa: E402
from tests import gen  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


class Writer:
    """Cases of one op. An array equal to one stored earlier (same dtype, shape
    and bytes) is stored once; later cases hold the string "@<key>" instead."""

    def __init__(self, name: str):
        self.name = name
        self.d: dict = {}
        self.seen: dict = {}
        self.n = 0

    def case(self, **arrays):
        for k, v in arrays.items():
            if v is None:
                continue
            v = np.asarray(v)
            key = f"c{self.n}.{k}"
            ident = (v.dtype.str, v.shape, hashlib.sha256(v.tobytes()).hexdigest())
            if v.size > 16 and ident in self.seen:
                self.d[key] = np.array("@" + self.seen[ident])
            else:
                self.seen.setdefault(ident, key)
                self.d[key] = v
        self.n += 1

    def save(self):
        self.d["ncases"] = np.array(self.n)
        np.savez_compressed(HERE / f"{self.name}.npz", **self.d)
        print(f"{self.name}: {self.n} cases, {(HERE / (self.name + '.npz')).stat().st_size} bytes")


# ---------------------------------------------------------------------------
# GEMM family
# ---------------------------------------------------------------------------

def linear(ref: Oracle):
    w8, w32 = Writer("linear8"), Writer("linear32")
    shapes = [(1, 1, 1), (3, 15, 5), (4, 16, 4), (5, 17, 33), (9, 33, 3), (33, 64, 17), (16, 384, 24),
              (40, 96, 70), (130, 64, 129)]
    for i, (M, K, N) in enumerate(shapes):
        for has_bias, asym in ((True, True), (False, True), (True, False), (False, False)):
            x, w, b, z, m, s = gen.linear_case(9000 + 31 * i + 2 * has_bias + asym, M, K, N,
                                               has_bias=has_bias, asym=asym, shift_lo=-3, shift_hi=40)
            m[: min(N, 2)] = [0x80000000, 0xFFFFFFFF][: min(N, 2)]
            w8.case(x=x, w=w, bias=b, wz=z, mult=m, shift=s, out=ref.linear8(x, w, b, z, m, s))
            x, w, b, z, m, s = gen.realistic_linear_case(9500 + 31 * i + 2 * has_bias + asym, M, K, N,
                                                         has_bias=has_bias, asym=asym)
            w8.case(x=x, w=w, bias=b, wz=z, mult=m, shift=s, out=ref.linear8(x, w, b, z, m, s))
        # Linear32 shifts in [0, 40]: the reference shifts a 64-bit value, and
        # counts at or above 64 are undefined in C++
        x, w, b, z, m, s = gen.linear_case(9900 + i, M, K, N, shift_lo=0, shift_hi=40)
        w32.case(x=x, w=w, bias=b, wz=z, mult=m, shift=s, out=ref.linear32(x, w, b, z, m, s))
        x, w, b, z, m, s = gen.realistic_linear_case(9950 + i, M, K, N)
        s[:] = np.arange(N) % 4
        w32.case(x=x, w=w, bias=b, wz=z, mult=m, shift=s, out=ref.linear32(x, w, b, z, m, s))
    w8.save()
    w32.save()


def classifier(ref: Oracle):
    w = Writer("classifier")
    r = gen.rng(7000)
    for M, K, N in ((1, 40, 257), (3, 64, 100), (2, 384, 1000)):
        x = gen.i8(r, (1, M, K))
        e = gen.i8(r, (N, K), -127, 127)
        for mult, shift in ((0x80000000, 0), (int(r.integers(0, 2**32)), 3), (7, -2), (1, 33),
                            (int(r.integers(2**30, 2**31)), 9)):
            w.case(x=x, w=e, mult=np.uint32(mult), shift=np.int8(shift),
                   out=ref.classifier(x, e, mult, shift))
    w.save()


def conv1d(ref: Oracle):
    w = Writer("conv1d")
    geoms = [(1, 1, 1, 1, 1, 1, 0), (2, 3, 10, 4, 3, 1, 1), (1, 5, 17, 6, 3, 2, 1), (1, 4, 9, 3, 5, 2, 2),
             (2, 8, 31, 5, 3, 3, 0), (1, 80, 40, 32, 3, 1, 1), (2, 32, 40, 48, 3, 2, 1)]
    for i, (B, Cin, Tin, Cout, ks, stride, pad) in enumerate(geoms):
        r = gen.rng(7100 + i)
        x = gen.i8(r, (B, Cin, Tin))
        wt = gen.i8(r, (Cout, Cin * ks))
        bias = r.integers(-2**31, 2**31, size=Cout, dtype=np.int64).astype(np.int32)
        for mult, shift in ((0x80000000, 0), (int(r.integers(0, 2**32)), 7), (5, -9), (2**32 - 1, 40)):
            for b in (bias, None):
                w.case(x=x, w=wt, bias=b, mult=np.uint32(mult), shift=np.int8(shift),
                       stride=np.int64(stride), padding=np.int64(pad),
                       out=ref.conv1d(x, wt, b, mult, shift, stride, pad))
    w.save()


# ---------------------------------------------------------------------------
# row / element ops
# ---------------------------------------------------------------------------

def layernorm(ref: Oracle):
    w = Writer("layernorm32")
    for hidden in (384, 512, 768, 1024, 1280):
        for spread in (0, 50, 4000, 16383):
            x, g, b, lm, ls, om, os_ = gen.ln_case(7200 + hidden + spread, 9, hidden, spread)
            for params in ((lm, ls, om, os_), (255, -20, 0xFFFFFFFF, -1), (1, 0, 1, 40)):
                for beta in (b, None):
                    w.case(x=x, gamma=g, beta=beta, ln_m=np.uint8(params[0]), ln_s=np.int8(params[1]),
                           out_m=np.uint32(params[2]), out_s=np.int8(params[3]),
                           out=ref.layernorm32(x, g, beta, *params))
    w.save()


def rsqrt(ref: Oracle):
    w = Writer("rsqrt")
    r = gen.rng(7300)
    x = np.concatenate([np.arange(0, 3000, dtype=np.int32),
                        r.integers(-2**31, 2**31, 3000, dtype=np.int64).astype(np.int32),
                        (2 ** r.uniform(0, 31, 3000)).astype(np.int64).astype(np.int32),
                        np.array([2**31 - 1, -2**31, 2**30, 2**30 - 1, -1], np.int32)])
    for off in (0, 1, 12, 13, 15, 16, 29):
        w.case(x=x, offset=np.uint32(off), out=ref.rsqrt(x, off))
    w.save()


def gelu(ref: Oracle):
    w = Writer("gelu")
    r = gen.rng(7400)
    x = np.arange(-128, 128, dtype=np.int8).repeat(9).reshape(-1, 36)
    for pc in ((True, True), (False, True), (True, False), (False, False)):
        for _ in range(2):
            lut, im, is_, om, os_ = gen.gelu_params(r, 36, *pc)
            is_ = is_.copy()
            is_[0] = -5
            if is_.size > 1:
                is_[1] = 40
            w.case(x=x, lut=lut, luti_m=im, luti_s=is_, luto_m=om, luto_s=os_,
                   out=ref.gelu(x, lut, im, is_, om, os_))
    w.save()


def residual15(ref: Oracle):
    w = Writer("residual15")
    r = gen.rng(7500)
    br = r.integers(-2**31, 2**31, size=4000, dtype=np.int64).astype(np.int32)
    res = r.integers(-32768, 32768, size=4000).astype(np.int16)
    br[:4] = [2**31 - 1, -2**31, 16383 << 15, -(16384 << 15)]
    br[4:1004] = r.integers(-2**22, 2**22, size=1000)
    for m in (0, 1, 2, 32768, 65535, 30000):
        w.case(branch=br, residual=res, mult=np.uint16(m), out=ref.residual15(br, res, m))
    w.save()


def add_requant15(ref: Oracle):
    w = Writer("add_requant15")
    r = gen.rng(7600)
    x = gen.i8(r, (2, 9, 24))
    a = gen.i8(r, (9, 24))
    for mc, sc in ((1, 1), (24, 24), (1, 24), (24, 1)):
        for _ in range(2):
            m = r.integers(0, 65536, size=mc).astype(np.uint16)
            s = r.integers(-4, 40, size=sc).astype(np.int8)
            w.case(x=x, addend=a, mult=m, shift=s, out=ref.add_requant15(x, a, m, s))
    w.save()


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def attention(ref: Oracle):
    w = Writer("attention")
    shapes = [(1, 1, 1, 1, 1), (1, 2, 3, 5, 4), (2, 3, 4, 4, 16), (1, 1, 1, 33, 64), (2, 2, 7, 9, 17),
              (1, 2, 16, 16, 64), (1, 2, 1, 40, 64), (1, 1, 3, 3, 96), (1, 1, 40, 40, 64),
              (1, 2, 2, 70, 128)]
    params = [None, (255, -3, 1, 1, 40), (1, 40, 13, 255, -2), (200, 0, 8, 17, 0)]
    for i, (B, H, Tq, Tk, D) in enumerate(shapes):
        q, k, v, qm, qs, f, am, as_ = gen.attn_case(7700 + i, B, H, Tq, Tk, D)
        for masked in (False, True):
            mask = gen.causal_mask(Tq, Tk) if masked and Tk >= Tq else None
            if masked and mask is None:
                continue
            for prm in params:
                qm_, qs_, f_, am_, as__ = (qm, qs, f, am, as_) if prm is None else prm
                qk, rm = ref.qk_requant_rowmax(q, k, mask, qm_, qs_)
                p, rs = ref.shift_exp(qk, rm, mask, f_)
                off = 16 if prm is None else (0, 16, 29)[i % 3]
                out = ref.pv_norm_requant(p, v, rs, am_, as__, off)
                w.case(q=q, k=k, v=v, mask=mask, qk_m=np.uint8(qm_), qk_s=np.int32(qs_),
                       frac_bits=np.int32(f_), av_m=np.uint8(am_), av_s=np.int8(as__),
                       rsqrt_offset=np.uint32(off), qk=qk, rmp1=rm, p=p, row_sum=rs, out=out)
    # the int16 row-max wrap corner: every score saturates at 32767, so
    # row_max + 1 wraps to -32768 and x_sub = 0 gives P = 2^f >> (f - 7) = 128
    q = np.full((1, 1, 2, 64), 127, np.int8)
    k = np.full((1, 1, 5, 64), 127, np.int8)
    v = gen.i8(gen.rng(7790), (1, 1, 64, 5))
    qk, rm = ref.qk_requant_rowmax(q, k, None, 255, 0)
    p, rs = ref.shift_exp(qk, rm, None, 9)
    out = ref.pv_norm_requant(p, v, rs, 100, 6, 16)
    w.case(q=q, k=k, v=v, qk_m=np.uint8(255), qk_s=np.int32(0), frac_bits=np.int32(9),
           av_m=np.uint8(100), av_s=np.int8(6), rsqrt_offset=np.uint32(16), qk=qk, rmp1=rm, p=p,
           row_sum=rs, out=out)
    w.save()


# ---------------------------------------------------------------------------
# digests at full model shapes (inputs from tests/gen.py seeds)
# ---------------------------------------------------------------------------

def digests(ref: Oracle) -> dict:
    D = {}
    # Whisper-large QKV / FC1 / FC2 GEMM slices (M rows of the real K, N)
    gemms = {"qkv_large": (64, 1280, 3840), "fc1_large": (32, 1280, 5120),
             "fc2_large": (32, 5120, 1280), "qkv_base": (96, 512, 1536)}
    for i, (name, (M, K, N)) in enumerate(gemms.items()):
        seed = 11000 + i
        x, w, b, z, m, s = gen.realistic_linear_case(seed, M, K, N)
        D[f"linear8.{name}"] = {"seed": seed, "shape": [M, K, N],
                                "sha256": sha(ref.linear8(x, w, b, z, m, s))}
        x, w, b, z, m, s = gen.realistic_linear_case(seed + 100, M, K, N)
        s[:] = np.arange(N) % 4
        D[f"linear32.{name}"] = {"seed": seed + 100, "shape": [M, K, N], "shift_mod": 4,
                                 "sha256": sha(ref.linear32(x, w, b, z, m, s))}
    # LayerNorm over 1500 rows of every width
    for hidden in (384, 512, 768, 1024, 1280):
        x, g, b, lm, ls, om, os_ = gen.ln_case(12000 + hidden, 1500, hidden, 3000)
        D[f"layernorm32.{hidden}"] = {"seed": 12000 + hidden, "rows": 1500, "hidden": hidden,
                                      "spread": 3000,
                                      "sha256": sha(ref.layernorm32(x, g, b, lm, ls, om, os_))}
    # encoder self-attention, one head at 1500 frames; decoder cross-attention step
    for name, (B, H, Tq, Tk, Dh) in {"enc_1500": (1, 1, 1500, 1500, 64),
                                     "cross_step": (2, 4, 1, 1500, 64),
                                     "enc_1500_d96": (1, 1, 1500, 1500, 96)}.items():
        seed = 13000 + Tq + Dh + B
        q, k, v, qm, qs, f, am, as_ = gen.attn_case(seed, B, H, Tq, Tk, Dh)
        out = ref.attention(q, k, v, None, qm, qs, f, am, as_, 16)
        D[f"attention.{name}"] = {"seed": seed, "shape": [B, H, Tq, Tk, Dh], "sha256": sha(out)}
    return D


def model_tiny():
    """End-to-end: a 1+1-layer model at d=384 with 4 heads (head dim 96) over
    200 audio frames, built by the package's seeded synthetic calibrator and
    run through the reference kernels along the reference dataflow."""
    import __graft_entry__
    from oracle.model_oracle import OracleWhisper

    iw = __graft_entry__.load_package()
    dims = iw.ModelDimensions(n_mels=80, n_audio_ctx=100, n_audio_state=384, n_audio_head=4,
                              n_audio_layer=1, n_vocab=1000, n_text_ctx=48, n_text_state=384,
                              n_text_head=4, n_text_layer=1)
    # decoder MLP outputs scaled down so that the argmax follows the input
    params = iw.synth.calibrated_int_params(dims, seed=4321, calib_ctx=100, decoder_mlp_scale=0.1)
    mel = iw.synth.synthetic_mel(2, dims.n_mels, 2 * dims.n_audio_ctx, seed=77)
    ref = OracleWhisper(dims, params, kind="ref")
    x = ref.encoder_input(mel)
    feats = ref.encoder(x)
    # a different seeded random prompt per row
    prompt = iw.synth.prompt_tokens(2, dims.n_vocab, seed=78)
    toks, logits = ref.greedy(feats, prompt, 12, return_logits=True)
    # teacher-forced steps: 16 seeded random input tokens per row fed through
    # the cache, so that the inputs, and with them the argmax ids, vary from
    # step to step (greedy decoding of a random-weight model repeats a token)
    forced = np.random.default_rng(79).integers(0, dims.n_vocab, size=(2, 16)).astype(np.int64)
    f_argmax, f_logits = ref.forced(feats, prompt, forced)
    out = {"dims": np.array([dims.n_mels, dims.n_audio_ctx, dims.n_audio_state, dims.n_audio_head,
                             dims.n_audio_layer, dims.n_vocab, dims.n_text_ctx, dims.n_text_state,
                             dims.n_text_head, dims.n_text_layer], np.int64),
           "mel_int8": x, "encoder_out": feats, "prompt": prompt, "tokens": toks, "logits": logits,
           "forced": forced, "forced_argmax": f_argmax, "forced_logits": f_logits}
    for k, v in params.items():
        out["param." + k] = v
    np.savez_compressed(HERE / "model_tiny.npz", **out)
    print(f"model_tiny: tokens {toks.tolist()}, forced argmax {f_argmax.tolist()}, "
          f"{(HERE / 'model_tiny.npz').stat().st_size} bytes")


def main():
    if not available("ref"):
        raise SystemExit("oracle/_ref is not built: run `make -C oracle ref` where the reference "
                         "tree is present")
    ref = Oracle("ref")
    linear(ref)
    classifier(ref)
    conv1d(ref)
    layernorm(ref)
    rsqrt(ref)
    gelu(ref)
    residual15(ref)
    add_requant15(ref)
    attention(ref)
    with open(HERE / "digests.json", "w") as f:
        json.dump(digests(ref), f, indent=1, sort_keys=True)
    print("digests.json written")
    model_tiny()


if __name__ == "__main__":
    import sys

    if sys.argv[1:] == ["model_tiny"]:  # only the end-to-end fixture
        model_tiny()
    else:
        main()
