"""GPU parity of the device-resident decode step (hs_decode_step_device,
src/engine.ts:1626-1644) against the oracle's decode loop: every step's
tokens, the stop check, rows that stay done, and the final history rings and
lengths, with all steps enqueued before one synchronisation.  Histories wrap
their rings (the repetition window read across the wrap), presence /
frequency rows count the ring's ids, and every routing of the sampler (row
kernel whole or split, chunk kernels, large-k pre-pass) reads the rings."""
import numpy as np
import pytest

from hachiue_amd import hip
from hachiue_amd.decode import DecodeState
from oracle import pyoracle as o

pytestmark = pytest.mark.gpu

CFGS = [
    dict(temperature=0.0),                                            # sampler.ts greedy
    dict(temperature=0.0, repetitionPenalty=1.3),
    dict(temperature=0.7, topK=40, topP=0.9, repetitionPenalty=1.1),
    dict(temperature=1.0, topK=200, topP=0.95, presencePenalty=0.5, frequencyPenalty=0.3),
    dict(temperature=0.8, topK=0, topP=0.97, minP=0.05, repetitionPenalty=1.2),
    dict(temperature=0.9, topK=2000, topP=0.9, repetitionPenalty=1.05),   # large-k path
]


def run_decode(sampler, V, prompts, stop_ids, cfgs, n_steps, ring_cap, seed, plant=None):
    rows = len(prompts)
    rng = np.random.default_rng(seed)
    base = [(rng.standard_normal((rows, V)) * 2.0).astype(np.float32) for _ in range(n_steps)]
    if plant:   # (step, row, id): that row's maximum at that step
        for s, r, t in plant:
            base[s][r, t] = np.float32(50.0)
    u = rng.random((n_steps, rows))
    print(f"[gpu] decode V={V} rows={rows} steps={n_steps} cap={ring_cap} seed={seed}", flush=True)
    ref_in = [b.copy() for b in base]
    ref = o.decode_loop(ref_in, V, prompts, stop_ids, cfgs, u, ring_cap=ring_cap)
    st = DecodeState(sampler, prompts, stop_ids, ring_cap=ring_cap)
    d_l = hip.DeviceArray.from_numpy(np.stack(base))
    d_u = hip.DeviceArray.from_numpy(u)
    d_t = hip.DeviceArray((n_steps, rows), np.int32)
    for s in range(n_steps):
        st.step(d_l.addr + s * rows * V * 4, V, V, cfgs, d_u.addr + s * rows * 8,
                d_t.addr + s * rows * 4)
    hip.synchronize()
    tokens = d_t.download()
    got = d_l.download()
    # A draw within 1e-6 of a cumulative boundary (or a top-p cut within 1e-6)
    # may go either way; the row's later steps then see another history.
    diverged = {}
    for s in range(n_steps):
        res = ref.steps[s]
        for r in range(rows):
            if r in diverged:
                continue
            ok_logits = np.array_equal(got[s, r].view(np.uint32), ref_in[s][r].view(np.uint32))
            assert ok_logits, f"step {s} row {r}: penalised logits differ"
            if tokens[s, r] != ref.tokens[s, r]:
                near = res.draw_margin[r] < 1e-6 or res.topp_margin[r] < 1e-6
                assert near, f"step {s} row {r}: token {tokens[s, r]} != {ref.tokens[s, r]}"
                diverged[r] = s
    assert len(diverged) <= max(1, rows // 20), diverged
    done, lens = st.finished(), st.lengths()
    for r in range(rows):
        if r in diverged:
            continue
        assert bool(done[r]) == ref.done[r]
        assert lens[r] == len(ref.histories[r])
        assert st.history(r).tolist() == ref.histories[r][-ring_cap:]
    print(f"[gpu] decode ok, boundary divergences {diverged}", flush=True)
    st.free()
    return ref


@pytest.mark.parametrize("V", [151936, 32000])
def test_decode_steps_match_oracle(any_sampler, V):
    rng = np.random.default_rng(V)
    prompts = [[], rng.integers(0, V, 5).tolist(), rng.integers(0, V, 200).tolist(),
               rng.integers(0, V, 1000).tolist(), rng.integers(0, 64, 300).tolist(),
               rng.integers(0, V, 130).tolist()]
    stop = [7, 11]
    plant = [(3, 0, 7), (5, 2, 11), (2, 4, 3)]   # rows 0 and 2 stop, row 4 draws id 3
    run_decode(any_sampler, V, prompts, stop, CFGS, 8, 256, seed=V + 1, plant=plant)


def test_decode_exact_window_ring(sampler):
    """ring_cap 128: the ring is exactly the repetition window; a prompt of
    1000 ids has wrapped it many times."""
    V = 4096
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, 32, 1000).tolist() for _ in range(4)]
    cfgs = [dict(temperature=0.0, repetitionPenalty=2.0),
            dict(temperature=0.6, topK=20, repetitionPenalty=1.5),
            dict(temperature=0.0, repetitionPenalty=0.5),
            dict(temperature=1.0, topK=64, topP=0.8, repetitionPenalty=1.3)]
    run_decode(sampler, V, prompts, [], cfgs, 12, 128, seed=6)


def test_decode_many_rows(sampler):
    """300 rows: the row kernel takes whole rows (no split)."""
    V = 32000
    rng = np.random.default_rng(8)
    prompts = [rng.integers(0, V, int(n)).tolist() for n in rng.integers(0, 400, 300)]
    cfgs = [CFGS[i % 5] for i in range(300)]
    run_decode(sampler, V, prompts, [1, 2, 3], cfgs, 3, 256, seed=9)


def test_decode_empty_vocabulary(sampler):
    """vocab 0: every draw is 0 (src/sampler.ts reads no logit); the stop
    check and the append still run."""
    st = DecodeState(sampler, [[5], [], [1, 2, 3]], [0], ring_cap=128)
    st2 = DecodeState(sampler, [[5], [], [1, 2, 3]], [], ring_cap=128)
    d_u = hip.DeviceArray.from_numpy(np.zeros(3))
    d_t = hip.DeviceArray(3, np.int32)
    print("[gpu] decode vocab 0", flush=True)
    st.step(0, 0, 0, [None] * 3, d_u.addr, d_t.addr)
    st.step(0, 0, 0, [None] * 3, d_u.addr, d_t.addr)
    hip.synchronize()
    assert d_t.download().tolist() == [-1, -1, -1]
    assert st.finished().tolist() == [True, True, True]
    assert st.lengths().tolist() == [1, 0, 3]
    st2.step(0, 0, 0, [None] * 3, d_u.addr, d_t.addr)
    hip.synchronize()
    assert d_t.download().tolist() == [0, 0, 0]
    assert st2.lengths().tolist() == [2, 1, 4]
    assert st2.history(2).tolist() == [1, 2, 3, 0]
    st.free()
    st2.free()


def test_decode_rejects_bad_arguments(sampler):
    from hachiue_amd.sampler import SamplerError
    st = DecodeState(sampler, [[1, 2]], [], ring_cap=128)
    d_l = hip.DeviceArray.from_numpy(np.zeros((1, 16), np.float32))
    d_u = hip.DeviceArray.from_numpy(np.zeros(1))
    d_t = hip.DeviceArray(1, np.int32)
    with pytest.raises(SamplerError):
        sampler.decode_step_device(d_l.addr, 1, 16, 16, st.ring.addr, 64, st.len.addr,
                                   st.done.addr, None, 0, [None], d_u.addr, d_t.addr)
    with pytest.raises(SamplerError):
        sampler.decode_step_device(d_l.addr, 1, 16, 16, st.ring.addr, 128, st.len.addr,
                                   st.done.addr, None, 3, [None], d_u.addr, d_t.addr)
    st.free()


def test_decode_large_k_ties_resolved(sampler):
    """Large-k rows whose draw lands in a group of equal logits are resolved
    by the slot replay (its slots in LDS at k = 5000, in device memory at
    k = 20000) inside a decode step: the tokens, histories and lengths equal
    the oracle's decode loop."""
    V = 40000
    logits = np.zeros((3, V), np.float32)
    logits[1] = np.round(np.random.default_rng(3).standard_normal(V) * 2)
    logits[2] = np.random.default_rng(4).standard_normal(V).astype(np.float32)
    cfgs = [dict(temperature=1.0, topK=5000.0, topP=0.95),
            dict(temperature=0.8, topK=20000.0, topP=0.9),
            dict(temperature=0.0)]
    uni = np.array([0.999, 0.37, 0.5])
    st = DecodeState(sampler, [[1, 2], [3], [4]], [], ring_cap=128)
    d_l = hip.DeviceArray.from_numpy(logits)
    d_u = hip.DeviceArray.from_numpy(uni)
    d_t = hip.DeviceArray(3, np.int32)
    print("[gpu] decode large-k ties", flush=True)
    st.step(d_l.addr, V, V, cfgs, d_u.addr, d_t.addr)
    hip.synchronize()
    tok = d_t.download().tolist()
    want = o.sample_batch(logits.copy(), V, None, None, cfgs, uni).token
    assert tok == list(want)
    assert st.lengths().tolist() == [3, 2, 2]
    assert st.history(0).tolist() == [1, 2, tok[0]]
    assert st.history(1).tolist() == [3, tok[1]]
    assert st.finished().tolist() == [False, False, False]
    st.free()


def test_decode_large_k_ties_beyond_2_19_resolved(sampler):
    """Top-k above 2^19 on a vocabulary larger than that, with the draw in
    a group of equal logits: the device-memory replay orders the group
    (src/sampler.ts:55-74), and the decode step appends the oracle's token."""
    V = 600000
    logits = np.zeros((2, V), np.float32)
    logits[1] = np.random.default_rng(3).standard_normal(V).astype(np.float32)
    cfgs = [dict(temperature=1.0, topK=550000.0, topP=0.95), dict(temperature=0.0)]
    uni = np.array([0.999, 0.5])
    st = DecodeState(sampler, [[1, 2], [3]], [], ring_cap=128)
    d_l = hip.DeviceArray.from_numpy(logits)
    d_u = hip.DeviceArray.from_numpy(uni)
    d_t = hip.DeviceArray(2, np.int32)
    print("[gpu] decode large-k ties beyond 2^19", flush=True)
    st.step(d_l.addr, V, V, cfgs, d_u.addr, d_t.addr)
    hip.synchronize()
    tok = d_t.download().tolist()
    want = o.sample_batch(logits.copy(), V, None, None, cfgs, uni).token
    assert tok == list(want)
    assert st.lengths().tolist() == [3, 2]
    assert st.history(0).tolist() == [1, 2, tok[0]]
    assert st.history(1).tolist() == [3, tok[1]]
    st.free()


def test_decode_unresolved_row_keeps_state(sampler):
    """A row the sampler leaves unresolved (HS_ROW_UNSUPPORTED, token -1:
    top-k above the replay's 2^24 slots on a vocabulary larger than that,
    with the draw in a group of equal logits) reports -1 in a decode step
    and keeps its history, length and done flag, while the other row
    advances."""
    V = (1 << 24) + 1024
    logits = np.zeros((2, V), np.float32)
    logits[1, ::4099] = np.random.default_rng(3).standard_normal(logits[1, ::4099].size)
    cfgs = [dict(temperature=1.0, topK=float((1 << 24) + 1), topP=0.95), dict(temperature=0.0)]
    st = DecodeState(sampler, [[1, 2], [3]], [], ring_cap=128)
    d_l = hip.DeviceArray.from_numpy(logits)
    d_u = hip.DeviceArray.from_numpy(np.array([0.999, 0.5]))
    d_t = hip.DeviceArray(2, np.int32)
    print("[gpu] decode unresolved row", flush=True)
    st.step(d_l.addr, V, V, cfgs, d_u.addr, d_t.addr)
    hip.synchronize()
    tok = d_t.download().tolist()
    # the greedy row alone through the oracle
    want = o.sample_batch(logits[1:].copy(), V, None, None, cfgs[1:], np.array([0.5])).token
    assert tok[1] == want[0]
    assert tok[0] == -1
    assert st.lengths().tolist() == [2, 2]
    assert st.history(0).tolist() == [1, 2]
    assert st.finished().tolist() == [False, False]
    assert st.history(1).tolist() == [3, tok[1]]
    st.free()
