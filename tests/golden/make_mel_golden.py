"""Write tests/golden/mel_filters_n400.npz: the reference's shipped mel filterbanks
(i_whisper/assets/mel_filters.npz, librosa.filters.mel(sr=16000, n_fft=400,
n_mels=80 / 128)), the fixed point that pins the package's filterbank
restatement. Run from the repository root where /root/reference exists;
np.load with allow_pickle=False executes nothing from the file."""
from pathlib import Path

import numpy as np

SRC = Path("/root/reference/i_whisper/assets/mel_filters.npz")
OUT = Path(__file__).resolve().parent / "mel_filters_n400.npz"

with np.load(SRC, allow_pickle=False) as f:
    np.savez_compressed(OUT, mel_80=f["mel_80"], mel_128=f["mel_128"])
print("wrote", OUT, OUT.stat().st_size, "bytes")
