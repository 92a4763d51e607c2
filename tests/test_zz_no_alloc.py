"""iw_log_mel_noalloc: the log-mel entry point that allocates nothing (its block
maxima live in a fixed per-GPU device array) against iw_log_mel with a caller
workspace, called through the C ABI: two calls in a row, the second on a
smaller input, bit-identical outputs; inputs beyond the fixed array are
rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _tables(iw, n_mels):
    return iw.audio._FrontEnd(n_mels, torch.device("cuda:0"))


def _run(iw, fe, audio, noalloc):
    B, L = audio.shape
    T = L // 160
    out = torch.full((B, fe.n_mels, T), float("nan"), dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    head = (audio.data_ptr(), B, L, L, fe.twiddle.data_ptr(), fe.window.data_ptr(), fe.start.data_ptr(),
            fe.len.data_ptr(), fe.off.data_ptr(), fe.w.data_ptr(), fe.n_taps, fe.n_mels, out.data_ptr(),
            fe.n_mels * T)
    if noalloc:
        iw._lib.call("iw_log_mel_noalloc", *head, st)
    else:
        ws = torch.empty(iw._lib.value("iw_log_mel_scratch_floats", B, L), dtype=torch.float32, device="cuda")
        iw._lib.call("iw_log_mel", *head, ws.data_ptr(), st)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_workspace_entry_point(iw, gpu):
    fe = _tables(iw, 80)
    g = torch.Generator(device="cuda").manual_seed(3)
    # first call: 6 loud rows of 30 s (282 block maxima); second: 2 quiet rows
    # of 7.3 s, so the larger maxima the first call left in the array would
    # change the second call's floor if it read any of them
    a1 = torch.randn((6, 480000), generator=g, device="cuda", dtype=torch.float32) * 0.1
    a2 = torch.randn((2, 116800), generator=g, device="cuda", dtype=torch.float32) * 0.01
    for a in (a1, a2):
        print("no-alloc log-mel:", tuple(a.shape), flush=True)
        want = _run(iw, fe, a, noalloc=False)
        got = _run(iw, fe, a, noalloc=True)
        assert not np.isnan(got).any()
        assert np.array_equal(got, want)


def test_noalloc_128_mels_and_limit(iw, gpu):
    fe = _tables(iw, 128)
    g = torch.Generator(device="cuda").manual_seed(4)
    a = torch.randn((3, 48000), generator=g, device="cuda", dtype=torch.float32)
    assert np.array_equal(_run(iw, fe, a, noalloc=True), _run(iw, fe, a, noalloc=False))
    # the largest accepted batch of 30 s rows is 65536 // 47 = 1394; one more
    # row is refused on the host, before any launch
    L = 480000
    assert iw._lib.value("iw_log_mel_scratch_floats", 1394, L) <= 65536 < \
        iw._lib.value("iw_log_mel_scratch_floats", 1395, L)
    lib = iw._lib.load()
    out = torch.empty(1, dtype=torch.float32, device="cuda")
    rc = lib.iw_log_mel_noalloc(a.data_ptr(), 1395, L, L, fe.twiddle.data_ptr(), fe.window.data_ptr(),
                                fe.start.data_ptr(), fe.len.data_ptr(), fe.off.data_ptr(), fe.w.data_ptr(),
                                fe.n_taps, 128, out.data_ptr(), 128 * (L // 160),
                                torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"exceeds the fixed scratch" in lib.iw_last_error()
