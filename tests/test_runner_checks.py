"""Shape and dtype checks of the batched runners, before any device work: a
mel batch, audio features or a prompt that do not match the runner's batch
and sizes raise ValueError instead of reading or writing past the runner's
buffers."""
from types import SimpleNamespace

import pytest
import torch


def enc_stub():
    return SimpleNamespace(B=4, T=1500, enc=SimpleNamespace(n_mels=80))


def dec_stub(filters=None):
    return SimpleNamespace(B=4, Ta=1500, C=384, Tcap=448, hist_cols=448, filters=filters,
                           dec=SimpleNamespace(n_ctx=448, n_vocab=51865))


@pytest.mark.parametrize("shape,dtype", [((3, 80, 3000), torch.float32), ((5, 80, 3000), torch.float32),
                                         ((4, 128, 3000), torch.float32), ((4, 80, 2000), torch.float32),
                                         ((4, 80, 3000), torch.float16)])
def test_encoder_runner_rejects_mismatched_mel(iw, shape, dtype):
    with pytest.raises(ValueError):
        iw.EncoderRunner.__call__(enc_stub(), torch.zeros(shape, dtype=dtype))


@pytest.mark.parametrize("shape,dtype", [((3, 1500, 384), torch.int8), ((8, 1500, 384), torch.int8),
                                         ((4, 1000, 384), torch.int8), ((4, 1500, 512), torch.int8),
                                         ((4, 1500, 384), torch.int16)])
def test_decoder_runner_rejects_mismatched_audio(iw, shape, dtype):
    with pytest.raises(ValueError):
        iw.DecoderRunner.set_audio(dec_stub(), torch.zeros(shape, dtype=dtype))


def test_decoder_runner_rejects_cpu_audio(iw):
    with pytest.raises(ValueError, match="GPU"):
        iw.DecoderRunner.set_audio(dec_stub(), torch.zeros((4, 1500, 384), dtype=torch.int8))


@pytest.mark.parametrize("shape,steps", [((3, 3), 5), ((4,), 5), ((4, 0), 5), ((4, 3), 0), ((4, 3), 446)])
def test_decoder_runner_rejects_bad_prompt(iw, shape, steps):
    with pytest.raises(ValueError):
        iw.DecoderRunner.run(dec_stub(), torch.zeros(shape, dtype=torch.int64), steps)


def test_greedy_decode_rejects_runner_with_other_filters(iw):
    runner = dec_stub(filters=iw.LogitFilters(eot=50257))
    model = SimpleNamespace(decoder=SimpleNamespace(n_ctx=448, n_vocab=51865))
    prompt = torch.zeros((4, 3), dtype=torch.int64)
    with pytest.raises(ValueError, match="filters"):
        iw.greedy_decode(model, torch.zeros((4, 1500, 384), dtype=torch.int8), prompt, 5, runner=runner)
