"""Log-mel front end on the GPU (i_whisper/audio.py:216-267) and the
integer model's input quantisation (model_int.py:1265-1267).

``mel_filterbank`` restates the Slaney-style mel filterbank the reference takes
from librosa (``librosa.filters.mel(sr=16000, n_fft=N_FFT, n_mels)``, default
fmin = 0, fmax = sr/2, htk=False, norm="slaney"), computed in float64 and
returned as float32. ``log_mel_spectrogram`` runs the STFT (periodic Hann
window, centred frames with reflect padding), the power spectrum, the mel
projection, log10, the "max - 8" floor and the affine rescale in two HIP
kernels (``iw_log_mel``).
"""
from __future__ import annotations

from functools import lru_cache
from typing import Optional

import numpy as np
import torch

from . import _lib

SAMPLE_RATE = 16000
N_FFT = 512          # audio.py:19 (this model's front end uses 512, not 400)
HOP_LENGTH = 160
CHUNK_LENGTH = 30
N_SAMPLES = CHUNK_LENGTH * SAMPLE_RATE
N_FRAMES = N_SAMPLES // HOP_LENGTH


def _hz_to_mel(f):
    f = np.asarray(f, dtype=np.float64)
    f_sp = 200.0 / 3
    mels = f / f_sp
    min_log_hz = 1000.0
    min_log_mel = min_log_hz / f_sp
    logstep = np.log(6.4) / 27.0
    return np.where(f >= min_log_hz, min_log_mel + np.log(np.maximum(f, 1e-300) / min_log_hz) / logstep, mels)


def _mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    f_sp = 200.0 / 3
    freqs = f_sp * m
    min_log_hz = 1000.0
    min_log_mel = min_log_hz / f_sp
    logstep = np.log(6.4) / 27.0
    return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), freqs)


@lru_cache(maxsize=None)
def mel_filterbank(sr: int, n_fft: int, n_mels: int) -> np.ndarray:
    """[n_mels, 1 + n_fft // 2] float32 triangular filters on the Slaney mel
    scale, each scaled by 2 / (its bandwidth in Hz)."""
    fftfreqs = np.linspace(0, float(sr) / 2, int(1 + n_fft // 2), endpoint=True)
    mel_pts = np.linspace(_hz_to_mel(0.0), _hz_to_mel(sr / 2.0), n_mels + 2)
    mel_f = _mel_to_hz(mel_pts)
    fdiff = np.diff(mel_f)
    ramps = np.subtract.outer(mel_f, fftfreqs)
    # the filters are held in float32 from the start (each triangle rounded,
    # then scaled in float64 and rounded again), as librosa does
    weights = np.zeros((n_mels, len(fftfreqs)), dtype=np.float32)
    for i in range(n_mels):
        lower = -ramps[i] / fdiff[i]
        upper = ramps[i + 2] / fdiff[i + 1]
        weights[i] = np.maximum(0, np.minimum(lower, upper))
    enorm = 2.0 / (mel_f[2:n_mels + 2] - mel_f[:n_mels])
    weights *= enorm[:, None]
    return weights


class _FrontEnd:
    """Device tables for one n_mels: twiddles, window and the sparse filterbank."""

    def __init__(self, n_mels: int, device):
        fb = mel_filterbank(SAMPLE_RATE, N_FFT, n_mels)
        starts, lens, offs, w = [], [], [], []
        for row in fb:
            nz = np.nonzero(row)[0]
            s = int(nz[0]) if nz.size else 0
            e = int(nz[-1]) + 1 if nz.size else 0
            starts.append(s)
            lens.append(e - s)
            offs.append(len(w))
            w.extend(row[s:e].tolist())
        j = np.arange(N_FFT // 2, dtype=np.float64)
        tw = np.stack([np.cos(-2 * np.pi * j / N_FFT), np.sin(-2 * np.pi * j / N_FFT)], 1).astype(np.float32)
        i32 = dict(dtype=torch.int32, device=device)
        self.n_mels = n_mels
        self.n_taps = len(w)
        self.twiddle = torch.from_numpy(tw.reshape(-1)).to(device)
        self.window = torch.hann_window(N_FFT, dtype=torch.float32).to(device)
        self.start = torch.tensor(starts, **i32)
        self.len = torch.tensor(lens, **i32)
        self.off = torch.tensor(offs, **i32)
        self.w = torch.tensor(np.asarray(w, np.float32) if w else np.zeros(1, np.float32)).to(device)


_FRONT = {}


def log_mel_spectrogram(audio: torch.Tensor, n_mels: int = 80, padding: int = 0,
                        device: Optional[torch.device] = None) -> torch.Tensor:
    """log_mel_spectrogram (audio.py:216-267) on the GPU: float32 audio [samples]
    or [batch, samples] (16 kHz) -> [n_mels, frames] or [batch, n_mels, frames],
    frames = samples // 160. Each row of a batch is normalised by its own
    maximum, i.e. the batch equals the reference applied to each row."""
    if not torch.is_tensor(audio):
        audio = torch.from_numpy(np.asarray(audio, dtype=np.float32))
    if device is not None:
        audio = audio.to(device)
    if not audio.is_cuda:
        audio = audio.cuda()
    audio = audio.to(torch.float32)
    if padding > 0:
        audio = torch.nn.functional.pad(audio, (0, padding))
    single = audio.dim() == 1
    a = audio.reshape(1, -1) if single else audio.contiguous()
    B, L = a.shape
    key = (n_mels, a.device)
    if key not in _FRONT:
        _FRONT[key] = _FrontEnd(n_mels, a.device)
    fe = _FRONT[key]
    T = L // HOP_LENGTH
    out = torch.empty((B, n_mels, T), dtype=torch.float32, device=a.device)
    ws = torch.empty(B * ((T + 63) // 64), dtype=torch.float32, device=a.device)
    _lib.call("iw_log_mel", a.data_ptr(), B, L, L, fe.twiddle.data_ptr(), fe.window.data_ptr(),
              fe.start.data_ptr(), fe.len.data_ptr(), fe.off.data_ptr(), fe.w.data_ptr(), fe.n_taps, n_mels,
              out.data_ptr(), n_mels * T, ws.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return out[0] if single else out
