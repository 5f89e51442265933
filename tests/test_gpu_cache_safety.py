"""Context isolation and concurrency through the C ABI.

The reference's cache-safety test (tests/test_cache_safety.cpp:41-86) keeps
two different models live, frees and reloads one, and checks that every
context still replays its first results bit for bit; its weight caches are
keyed by raw tensor pointers (src/winograd.cpp:611-634,
src/directconv.cpp:1392-1445), which a freed-and-reused allocation could
alias.  Here each context owns its own device weight arena, so the same
sequence must give identical bits.  A context serialises concurrent calls
with its own mutex: two threads sharing one context must each get exactly
the sequential result.
"""
import os
import tempfile
import threading

import numpy as np
import pytest

from gpu_util import announce, device_ok
from vdamd import lib, synth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not device_ok(), reason="no HIP device")]

N3S = 48000


@pytest.fixture(scope="module")
def models():
    tmp = tempfile.mkdtemp()
    paths = {}
    paths["resnet_a"] = os.path.join(tmp, "resnet_a.gguf")
    synth.write_resnet34(paths["resnet_a"], seed=101)
    paths["resnet_b"] = os.path.join(tmp, "resnet_b.gguf")
    synth.write_resnet34(paths["resnet_b"], seed=202)
    paths["ecapa"] = os.path.join(tmp, "ecapa.gguf")
    synth.write_ecapa(paths["ecapa"], seed=303, channels=256, mfa=768)
    return paths


def test_two_models_free_and_reload_replay_bitwise(models):
    pcm = synth.clips(55, 4, N3S)
    announce("cache safety: two live models, free + reload, bitwise replay")
    a = lib.Context(models["resnet_a"])
    b = lib.Context(models["resnet_b"])
    ea0 = a.embed_batch(pcm)
    eb0 = b.embed_batch(pcm)
    # different weights give different embeddings: the contexts do not share state
    assert not np.array_equal(ea0, eb0)
    b.close()
    # a third, different family loads while `a` stays live
    c = lib.Context(models["ecapa"])
    ec0 = c.embed_batch(pcm)
    assert np.array_equal(a.embed_batch(pcm), ea0)
    # reload the freed model: its arena may reuse the freed addresses
    b2 = lib.Context(models["resnet_b"])
    assert np.array_equal(b2.embed_batch(pcm), eb0)
    assert np.array_equal(a.embed_batch(pcm), ea0)
    assert np.array_equal(c.embed_batch(pcm), ec0)
    # single-clip calls through the frozen ABI agree with the batch rows
    assert np.array_equal(b2.embed_pcm(pcm[2]), eb0[2])
    a.close()
    # after `a` is gone the others still replay
    assert np.array_equal(b2.embed_batch(pcm), eb0)
    assert np.array_equal(c.embed_batch(pcm), ec0)
    b2.close()
    c.close()


def test_two_threads_share_one_context(models):
    ctx = lib.Context(models["resnet_a"])
    jobs = [synth.clips(900 + i, 3, N3S) for i in range(2)]
    announce("cache safety: two threads on one context")
    want = [ctx.embed_batch(p) for p in jobs]
    got = [[None] * 4 for _ in jobs]
    errors = []

    def worker(t):
        try:
            for r in range(4):
                got[t][r] = ctx.embed_batch(jobs[t])
        except Exception as e:  # reported after the join
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
    for t in range(2):
        for r in range(4):
            assert np.array_equal(got[t][r], want[t]), f"thread {t} round {r}"
    ctx.close()
