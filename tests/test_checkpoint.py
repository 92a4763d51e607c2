"""Integer checkpoint I/O in the "i-whisper-int" v1 format (i_whisper/__init__.py:248-493):
layout, config and metadata, strict round trip of every state-dict tensor, the
loader's error cases, and (GPU) a loaded checkpoint reproducing the golden
end-to-end outputs."""
import json

import numpy as np
import pytest
import torch
from safetensors import safe_open

from tests.test_golden import model_fixture

# Whisper's ModelDimensions fields in declaration order (model_int.py's dataclass;
# config.json "dims" is asdict() of it)
DIM_FIELDS = ["n_mels", "n_audio_ctx", "n_audio_state", "n_audio_head", "n_audio_layer",
              "n_vocab", "n_text_ctx", "n_text_state", "n_text_head", "n_text_layer"]


@pytest.fixture(scope="module")
def tiny(iw):
    dims, params, z = model_fixture(iw)
    return dims, params, z, iw.Whisper_int.from_params(dims, params)


@pytest.fixture()
def saved(iw, tiny, tmp_path):
    ck = iw.checkpoint
    d = ck.save_int_model(tiny[3], tmp_path, "tiny1")
    return ck, d


def test_layout_config_and_metadata(tiny, saved):
    dims, params, _, _ = tiny
    ck, d = saved
    assert d.name == "iwhisper-tiny1" and sorted(p.name for p in d.iterdir()) == ["config.json",
                                                                                 "model.safetensors"]
    cfg = json.loads((d / "config.json").read_text())
    assert cfg["format"] == "i-whisper-int" and cfg["format_version"] == 1 and cfg["model_name"] == "tiny1"
    assert list(cfg["dims"]) == DIM_FIELDS
    assert [cfg["dims"][f] for f in DIM_FIELDS] == [int(getattr(dims, f)) for f in DIM_FIELDS]
    with safe_open(str(d / "model.safetensors"), "pt") as f:
        assert f.metadata() == {"format": "i-whisper-int", "format_version": "1"}
        keys = set(f.keys())
        assert keys == set(params)
        for k in keys:
            t = f.get_tensor(k)
            want = params[k]
            assert tuple(t.shape) == want.shape, k
            # same integer dtype as the state dict (uint16/uint32 included)
            assert str(t.dtype).replace("torch.", "") == str(want.dtype).replace("bool_", "bool"), k
            assert np.array_equal(t.to(torch.int64).numpy() if t.dtype in (torch.uint16, torch.uint32)
                                  else t.numpy(), want), k


def test_round_trip_every_tensor(tiny, saved):
    ck, d = saved
    loaded = ck.load_int_model(d, device="cpu")
    msgs = []
    ck.verify_int_model_roundtrip(tiny[3], loaded, streamer=msgs.append)
    assert "passed" in msgs[-1]
    dims2, params2 = ck.load_int_params(d)
    assert dims2 == tiny[0] and set(params2) == set(tiny[1])


def test_resolution_forms(tiny, saved):
    ck, d = saved
    by_alias = ck.load_int_model("tiny1", device="cpu", root=d.parent)
    by_file = ck.load_int_model(d / "model.safetensors", device="cpu")
    ck.verify_int_model_roundtrip(by_alias, by_file, streamer=lambda s: None)
    with pytest.raises(RuntimeError, match="Expected model.safetensors"):
        ck.load_int_model(d / "config.json", device="cpu")
    with pytest.raises(RuntimeError, match="not found"):
        ck.load_int_model("absent", device="cpu", root=d.parent)


def test_loader_rejects_other_formats(saved):
    ck, d = saved
    cfg = json.loads((d / "config.json").read_text())
    (d / "config.json").write_text(json.dumps({**cfg, "format_version": 2}))
    with pytest.raises(RuntimeError, match="format version"):
        ck.load_int_model(d, device="cpu")
    (d / "config.json").write_text(json.dumps({**cfg, "format": "other"}))
    with pytest.raises(RuntimeError, match="Unsupported model format"):
        ck.load_int_model(d, device="cpu")
    (d / "config.json").unlink()
    with pytest.raises(RuntimeError, match="Missing model configuration"):
        ck.load_int_model(d, device="cpu")


def test_verify_reports_changed_state(tiny, saved):
    ck, d = saved
    loaded = ck.load_int_model(d, device="cpu")
    key = "decoder.token_embedding.weight"
    with torch.no_grad():
        loaded.state_dict()[key].view(-1)[0] += 1
    with pytest.raises(AssertionError, match="value mismatch"):
        ck.verify_int_model_roundtrip(tiny[3], loaded, streamer=lambda s: None)
    with pytest.raises(TypeError):
        ck.save_int_model(torch.nn.Linear(2, 2), d.parent, "bad")


@pytest.mark.gpu
def test_loaded_checkpoint_reproduces_golden(iw, gpu, saved):
    ck, d = saved
    _, _, z = model_fixture(iw)
    model = ck.load_int_model(d, device="cuda")
    with torch.no_grad():
        feats = model.embed_audio(torch.from_numpy(z["mel_int8"]).cuda())
        toks, logits = iw.greedy_decode(model, feats, torch.from_numpy(z["prompt"]).cuda(),
                                        z["logits"].shape[1], keep_logits=True)
    assert np.array_equal(feats.cpu().numpy(), z["encoder_out"])
    assert np.array_equal(logits.cpu().numpy(), z["logits"])
    assert np.array_equal(toks.cpu().numpy(), z["tokens"])
