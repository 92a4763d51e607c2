"""Log-mel front end (audio.py:216-267, N_FFT = 512): the filterbank restatement
against the reference's shipped filterbanks (bit-exact), the CPU restatement's
STFT against an independent float64 DFT and a closed-form sinusoid, and the
HIP kernels against the restatement within float32 rounding."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import logmel_oracle as LM

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def A(iw):
    return iw.audio


def test_filterbank_matches_reference_assets(A):
    with np.load(GOLDEN / "mel_filters_n400.npz") as f:
        for n in (80, 128):
            got = A.mel_filterbank(16000, 400, n)
            assert got.dtype == np.float32 and np.array_equal(got, f[f"mel_{n}"]), n


def test_filterbank_shape_and_slaney_area(A):
    for n in (80, 128):
        fb = A.mel_filterbank(16000, 512, n).astype(np.float64)
        assert fb.shape == (n, 257) and (fb >= 0).all()
        peaks = fb.argmax(1)
        assert (np.diff(peaks) >= 0).all()
        # each triangle has unit area in Hz (Slaney normalisation) where it spans many bins
        wide = (fb > 0).sum(1) >= 12
        area = fb[wide].sum(1) * (16000 / 512)
        assert np.allclose(area, 1.0, rtol=0.05), area


def test_stft_power_matches_direct_dft():
    rng = np.random.default_rng(0)
    a = rng.standard_normal(16000 + 37).astype(np.float32)
    stft = torch.stft(torch.from_numpy(a), 512, 160, window=torch.hann_window(512), return_complex=True)
    p32 = (stft[..., :-1].abs() ** 2).numpy().astype(np.float64)
    p64 = LM.dft_power(a)
    assert p32.shape == p64.shape
    assert np.max(np.abs(p32 - p64)) <= 1e-4 * np.max(p64)


def test_sinusoid_closed_form():
    n = np.arange(8000)
    k0 = 32
    a = np.sin(2 * np.pi * k0 * n / 512).astype(np.float32)
    p = LM.dft_power(a)
    t = p.shape[1] // 2  # an interior frame
    assert int(np.argmax(p[:, t])) == k0
    # Hann-windowed sine at a bin centre: |X[k0]| = sum(w) / 2 = 128, the two
    # neighbours get half of that, every other bin nothing (float32 input)
    mag = np.sqrt(p[:, t])
    assert abs(mag[k0] - 128.0) < 1e-4 and np.allclose(mag[[k0 - 1, k0 + 1]], 64.0, atol=1e-4)
    others = np.delete(mag, [k0 - 1, k0, k0 + 1])
    assert others.max() < 1e-3


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("n_mels,length,batch", [(80, 480000, 2), (128, 480000, 1), (80, 16037, 3),
                                                 (128, 300, 1)])
def test_log_mel_matches_oracle(iw, gpu, A, n_mels, length, batch):
    print("log-mel", n_mels, length, batch, flush=True)
    rng = np.random.default_rng(length + n_mels)
    audio = (0.1 * rng.standard_normal((batch, length))).astype(np.float32)
    audio[0, : length // 3] *= 0.01  # a quiet stretch: the max - 8 floor bites
    got = A.log_mel_spectrogram(torch.from_numpy(audio).cuda(), n_mels=n_mels).cpu().numpy()
    fb = A.mel_filterbank(16000, 512, n_mels)
    for b in range(batch):
        want = LM.log_mel(audio[b], fb)
        assert got[b].shape == want.shape
        err = np.abs(got[b] - want)
        assert err.max() < 1e-4, err.max()
        # the int8 model input (x * alpha, round, clamp) agrees except at rounding ties
        alpha = 127.0 / 1.5
        qg = np.clip(np.rint(got[b] * np.float32(alpha)), -127, 127)
        qw = np.clip(np.rint(want * np.float32(alpha)), -127, 127)
        assert np.abs(qg - qw).max() <= 1 and (qg != qw).mean() < 1e-3


@pytest.mark.gpu
def test_log_mel_single_row_and_padding(iw, gpu, A):
    rng = np.random.default_rng(3)
    a = (0.05 * rng.standard_normal(40000)).astype(np.float32)
    got = A.log_mel_spectrogram(torch.from_numpy(a).cuda(), padding=480000 - 40000).cpu().numpy()
    want = LM.log_mel(np.pad(a, (0, 480000 - 40000)), A.mel_filterbank(16000, 512, 80))
    assert got.shape == (80, 3000) and np.abs(got - want).max() < 1e-4
