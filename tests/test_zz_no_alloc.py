"""The allocation-free entry point vx_sample_top_p_noalloc against the
existing device path of vx_sample_top_p, through the C ABI: the same code
and the same advanced generator state, on two calls in a row, the second
with fewer logits (the shared device staging keeps the first call's
contents, which must not leak into the second); sizes past the staging
array and bad parameters are rejected."""
import numpy as np
import pytest

import voxtral_amd as V
from vxtest import gpu_engine

pytestmark = pytest.mark.gpu


def test_noalloc_top_p_matches_the_engine_path():
    g = gpu_engine(n_layers=1, max_seq=16)
    try:
        rng = np.random.default_rng(21)
        state = 99
        for n, valid, scale, top_p, temp in ((8320, 8194, 3.0, 0.9, 0.8),
                                             (1000, 900, 0.5, 0.95, 1.3),
                                             (8320, 8194, 10.0, 0.5, 1.0),
                                             (64, 64, 1.0, 1.0, 0.7)):
            logits = (rng.standard_normal(n) * scale).astype(np.float32)
            ref, ref_state = g.sample_top_p(logits, valid, top_p, temp, state, on_device=True)
            got, got_state = V.sample_top_p_noalloc(logits, valid, top_p, temp, state)
            print(f"[noalloc] n {n}: engine {ref}, noalloc {got}", flush=True)
            assert got == ref and got_state == ref_state
            assert 1 <= got < valid
            state = ref_state
        # the masked entries stay masked when the staging held larger values
        # from a previous, longer call
        big = np.full(8320, 50.0, np.float32)
        V.sample_top_p_noalloc(big, 8194, 0.9, 0.8, 1)
        small = np.zeros(100, np.float32)
        for _ in range(5):
            code, state = V.sample_top_p_noalloc(small, 100, 0.9, 0.8, state)
            assert 1 <= code < 100
        with pytest.raises(V.VoxtralError, match="exceed the 9216 of the allocation-free"):
            V.sample_top_p_noalloc(np.zeros(9217, np.float32), 8194, 0.9, 0.8, 1)
        for bad in (dict(top_p=0.0), dict(top_p=float("nan")), dict(temperature=0.0)):
            kw = dict(top_p=0.9, temperature=0.8)
            kw.update(bad)
            with pytest.raises(V.VoxtralError, match="out of range"):
                V.sample_top_p_noalloc(np.zeros(100, np.float32), 100, kw["top_p"],
                                       kw["temperature"], 1)
    finally:
        g.destroy()
