"""Pins the oracle's FBank (oracle/oracle_fbank.c) before results are compared against it.

1. Golden vectors written by the reference's own src/fbank.cpp (tests/golden).
2. The reference library itself (oracle/_ref/libref.so) when it is built here.
3. What the mathematics fixes: frame count, povey window, mel filter geometry,
   CMN zero mean, FFT == naive DFT, a pure tone landing in its mel bin.
"""
import hashlib
import os

import numpy as np
import pytest

import pyoracle as O
from vdamd import synth


def _golden(golden_dir):
    return np.load(os.path.join(golden_dir, "fbank_golden.npz"))


def _cases(z):
    return sorted({k.split("/")[0] for k in z.files})


def _cfg(z, name):
    n_mels, n_fft, win, hop, cmn = z[name + "/cfg"]
    pre, lo, hi = z[name + "/cfgf"]
    return O.fbank_cfg(n_mels=int(n_mels), n_fft=int(n_fft), win=int(win), hop=int(hop),
                       preemph=float(pre), low=float(lo), high=float(hi), cmn=bool(cmn))


def golden_pcm(z, name):
    if name + "/pcm" in z.files:
        return z[name + "/pcm"]
    seed, n = z[name + "/seed"]
    pcm = synth.clip(int(seed), int(n))
    assert hashlib.sha256(pcm.tobytes()).digest() == z[name + "/sha256"].tobytes(), \
        "synthetic clip generator drifted from the golden input"
    return pcm


def test_oracle_matches_reference_goldens(golden_dir):
    z = _golden(golden_dir)
    names = _cases(z)
    assert len(names) >= 12
    for name in names:
        got = O.fbank(golden_pcm(z, name), _cfg(z, name))
        ref = z[name + "/fbank"]
        assert got.shape == ref.shape, name
        # same algorithm and precision as the reference: agreement to float rounding
        assert np.abs(got - ref).max() <= 1e-5, name


def test_oracle_matches_reference_library_random_lengths():
    if O.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    rng = np.random.default_rng(5)
    for n in (400, 401, 560, 1234, 16000, 48000, 64000):
        pcm = (rng.standard_normal(n) * 0.1).astype(np.float32)
        for cfg in (O.fbank_cfg(), O.fbank_cfg(cmn=False), O.fbank_cfg(n_fft=1024, win=800, hop=320)):
            got, ref = O.fbank(pcm, cfg), O.ref_fbank(pcm, cfg)
            assert got.shape == ref.shape
            if got.size:
                assert np.abs(got - ref).max() <= 1e-5


def test_frame_count_closed_form():
    cfg = O.fbank_cfg()
    for n, T in ((399, 0), (400, 1), (559, 1), (560, 2), (48000, 298), (64000, 398),
                 (160000, 998), (320000, 1998)):
        assert O.lib().orc_fbank_frames(n, cfg) == T


def test_povey_window_closed_form():
    w = O.povey(400)
    assert w[0] == 0.0 and w[-1] < 1e-12
    assert np.allclose(w, w[::-1], atol=1e-15)            # symmetric
    i = np.arange(400)
    hann = 0.5 - 0.5 * np.cos(2 * np.pi * i / 399)
    assert np.allclose(w, hann ** 0.85, rtol=1e-14, atol=0)
    assert np.all(w <= 1.0)


def test_mel_filter_geometry():
    cfg = O.fbank_cfg()
    fb = O.mel_filters(cfg)
    assert fb.shape == (80, 257)
    assert np.all(fb >= 0) and np.all(fb <= 1.0)
    assert np.all(fb[:, 256] == 0.0)                       # Nyquist bin carries no weight
    assert np.all(fb[:, 0] == 0.0)                         # DC (0 Hz) is below the 20 Hz band edge
    mel = lambda f: 1127.0 * np.log(1.0 + f / 700.0)      # noqa: E731
    edges = np.linspace(mel(20.0), mel(8000.0), 82)
    fbin = mel(np.arange(257) * 16000.0 / 512)
    for m in range(80):
        nz = np.nonzero(fb[m])[0]
        assert len(nz) >= 1
        # support strictly inside (left, right) edge, peak at the bin nearest the centre
        assert np.all(fbin[nz] > edges[m]) and np.all(fbin[nz] < edges[m + 2])
        peak = nz[np.argmax(fb[m, nz])]
        below = fbin <= edges[m + 1]
        assert peak in (np.max(np.nonzero(below)[0]), np.min(np.nonzero(~below)[0]))
    # adjacent triangles overlap so that interior bins sum to 1
    s = fb.sum(axis=0)
    inner = (fbin > edges[1]) & (fbin < edges[80])
    assert np.allclose(s[inner], 1.0, atol=1e-12)


def test_fft_equals_naive_dft():
    rng = np.random.default_rng(3)
    frame = rng.standard_normal(400).astype(np.float32)
    a = O.powspec(frame, 512)
    b = O.powspec(frame, 512, use_dft=True)
    c = np.abs(np.fft.rfft(frame.astype(np.float64), 512)) ** 2
    assert np.allclose(a, b, rtol=1e-9, atol=1e-9)
    assert np.allclose(a, c, rtol=1e-9, atol=1e-9)


def test_cmn_zero_mean_and_tone_bin():
    n = 48000
    t = np.arange(n) / 16000.0
    f0 = 1000.0
    pcm = (0.3 * np.sin(2 * np.pi * f0 * t)).astype(np.float32)
    f = O.fbank(pcm)
    assert np.abs(f.mean(axis=1)).max() < 1e-5
    raw = O.fbank(pcm, O.fbank_cfg(cmn=False))
    fb = O.mel_filters()
    k = int(round(f0 * 512 / 16000))
    expect = int(np.argmax(fb[:, k]))
    assert int(np.argmax(raw[:, 100])) in (expect - 1, expect, expect + 1)
    # CMN is exactly "subtract the per-bin time mean" of the raw features
    assert np.abs((raw - raw.mean(axis=1, keepdims=True)) - f).max() < 1e-5
