"""Semantic-code sampling: the device top-p kernel used by generate(), the
host implementation, and a restatement of the reference's JavaScript
sampleTopP (src/engine.ts:247-289: Float32Array storage, f64 arithmetic,
stable sort) pick the same index for the same uniform draw."""
import numpy as np
import pytest

from vxtest import gpu_engine

pytestmark = pytest.mark.gpu

GOLDEN = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


def splitmix_next(state):
    state = (state + GOLDEN) & M64
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31), state


def sample_top_p_js(logits, valid, top_p, temperature, state):
    """sampleTopP as the reference writes it, with the masking of generate()
    and Math.random() replaced by (z >> 11) * 2^-53."""
    lg = np.array(logits, np.float32, copy=True)
    lg[0] = -np.inf
    lg[valid:] = -np.inf
    n = lg.size
    scaled = np.empty(n, np.float32)
    for i in range(n):
        scaled[i] = np.float32(float(lg[i]) / temperature)
    max_v = max(float(v) for v in scaled)
    s = 0.0
    for i in range(n):
        scaled[i] = np.float32(np.exp(float(scaled[i]) - max_v))
        s += float(scaled[i])
    for i in range(n):
        scaled[i] = np.float32(float(scaled[i]) / s)
    order = sorted(range(n), key=lambda i: -float(scaled[i]))  # stable: ties keep index order
    cum, cutoff = 0.0, n
    for k, i in enumerate(order):
        cum += float(scaled[i])
        if cum >= top_p:
            cutoff = k + 1
            break
    resum = 0.0
    for k in range(cutoff):
        resum += float(scaled[order[k]])
    z, state = splitmix_next(state)
    r = (z >> 11) * 2.0 ** -53 * resum
    acc = 0.0
    for k in range(cutoff):
        acc += float(scaled[order[k]])
        if acc >= r:
            return order[k], state
    return order[0], state


@pytest.fixture(scope="module")
def eng():
    g = gpu_engine(n_layers=1, max_seq=64)
    yield g
    g.destroy()


def test_device_host_and_reference_agree(eng):
    rng = np.random.default_rng(0)
    same_dev, same_host, trials = 0, 0, 60
    state = 12345
    for t in range(trials):
        n = 8320
        scale = [0.05, 0.5, 3.0, 10.0][t % 4]
        logits = (rng.standard_normal(n) * scale).astype(np.float32)
        top_p, temp = [(0.9, 0.8), (0.5, 1.0), (1.0, 0.7), (0.95, 1.3)][t % 4]
        ref, st_ref = sample_top_p_js(logits, 8194, top_p, temp, state)
        dev, st_dev = eng.sample_top_p(logits, 8194, top_p, temp, state, on_device=True)
        host, st_host = eng.sample_top_p(logits, 8194, top_p, temp, state, on_device=False)
        assert st_dev == st_ref and st_host == st_ref
        same_dev += dev == ref
        same_host += host == ref
        assert 1 <= dev < 8194
        state = st_ref
    print(f"device {same_dev}/{trials}, host {same_host}/{trials} equal to the reference")
    assert same_host == trials
    # the device sums the masses exactly (integers), the reference in f64:
    # a pick can only differ where a running sum lies within f64 rounding of
    # the drawn threshold, which none of these draws does
    assert same_dev == trials


def test_ties_and_edge_cases(eng):
    state = 7
    # equal logits: ranks follow the index order, so the cumulative cutoff
    # and the draw are those of the sorted indices
    flat = np.zeros(1000, np.float32)
    for top_p in (0.1, 0.9, 1.0):
        for _ in range(5):
            ref, nxt = sample_top_p_js(flat, 900, top_p, 0.8, state)
            dev, _ = eng.sample_top_p(flat, 900, top_p, 0.8, state)
            assert dev == ref
            state = nxt
    # one dominant logit: always chosen
    peak = np.zeros(8320, np.float32)
    peak[4321] = 50.0
    for _ in range(5):
        dev, state = eng.sample_top_p(peak, 8194, 0.9, 0.8, state)
        assert dev == 4321
    # the masked index 0 and the padding are never chosen, whatever their logits
    lg = np.full(8320, -5.0, np.float32)
    lg[0] = 100.0
    lg[9000 % 8320] = 100.0
    lg[8200:] = 100.0
    for _ in range(5):
        dev, state = eng.sample_top_p(lg, 8194, 0.9, 0.8, state)
        assert 1 <= dev < 8194


def test_generate_device_and_host_sampling_agree():
    g = gpu_engine(n_layers=2, max_seq=128)
    try:
        toks = [1, 25, 24, 24, 35, 500, 24]
        a = g.generate(toks, 2, 0, None, 8, sampling="top_p", seed=11, ignore_eos=True)
        b = g.generate(toks, 2, 0, None, 8, sampling="top_p_host", seed=11, ignore_eos=True)
        assert a["semanticCodes"] == b["semanticCodes"]
        assert a["acousticCodes"] == b["acousticCodes"]
        # position after generate: prompt + kick + one step per later frame
        assert g.position == len(toks) + 1 + 7
    finally:
        g.destroy()
