"""CPU restatement of the log-mel front end (TEST INFRASTRUCTURE ONLY: the
tests compare iw_log_mel against it; nothing in the product imports it).

Follows i_whisper/audio.py:216-267 call by call with torch on the CPU:
torch.stft(audio, 512, 160, window=hann_window(512), return_complex=True)
(centred, reflect padding), |X|^2 without the last frame, filters @ power,
log10 of the clamp at 1e-10, max(., max - 8), / 4 + 1. The filterbank is
passed in (the package's restatement of librosa.filters.mel, pinned separately
against the reference's shipped filterbanks). ``dft_power`` is an independent
float64 DFT of the same frames, used to pin the STFT step.
"""
from __future__ import annotations

import numpy as np
import torch


def log_mel(audio: np.ndarray, filters: np.ndarray) -> np.ndarray:
    a = torch.from_numpy(np.asarray(audio, np.float32))
    window = torch.hann_window(512)
    stft = torch.stft(a, 512, 160, window=window, return_complex=True)
    magnitudes = stft[..., :-1].abs() ** 2
    mel_spec = torch.from_numpy(filters) @ magnitudes
    log_spec = torch.clamp(mel_spec, min=1e-10).log10()
    log_spec = torch.maximum(log_spec, log_spec.max() - 8.0)
    return (log_spec / 4.0 + 1.0).numpy()


def dft_power(audio: np.ndarray) -> np.ndarray:
    """|X[k, t]|^2 in float64 by direct DFT of the reflect-padded Hann frames."""
    a = np.asarray(audio, np.float64)
    n = np.arange(512)
    w = 0.5 - 0.5 * np.cos(2 * np.pi * n / 512)
    ap = np.pad(a, (256, 256), mode="reflect")
    T = len(a) // 160
    frames = np.stack([ap[t * 160:t * 160 + 512] * w for t in range(T)], 1)  # [512, T]
    k = np.arange(257)[:, None]
    basis = np.exp(-2j * np.pi * k * n[None, :] / 512)
    X = basis @ frames
    return np.abs(X) ** 2
