"""GPU parity of the large-k path (topK above 1024, up to Infinity): the
Gumbel workload (k = vocab, top-p 0.98), a partial top-k of a few thousand,
rows of equal logits, non-finite logits, and penalties routed through the
pre-pass.  Every call goes through the C ABI and is compared with the oracle;
no row of these inputs may be left unresolved (HS_ROW_UNSUPPORTED)."""
import numpy as np
import pytest

from hachiue_amd import workloads
from tests.gpu_util import compare, run_gpu, run_oracle

pytestmark = pytest.mark.gpu

HS_ROW_UNSUPPORTED = 0x10
HS_ROW_LARGE = 0x20
HS_ROW_TWO_PASS = 0x40


def _check(sampler, logits, vocab, hist_ids, hist_off, configs, uniforms, cap, label,
           want_cands=True):
    """want_cands=False asks for tokens, counts and cutoffs only: rows with
    k = vocab and no min-p then take the two-pass kernel."""
    got = run_gpu(sampler, logits, vocab, hist_ids, hist_off, configs, uniforms, cap,
                  want_cands=want_cands)
    want, want_logits = run_oracle(logits, vocab, hist_ids, hist_off, configs, uniforms, cap)
    unsupported = np.flatnonzero((got.flags & HS_ROW_UNSUPPORTED) != 0)
    assert unsupported.size == 0, f"{label}: rows left unresolved {unsupported[:10]}"
    assert (got.tokens >= 0).all(), f"{label}: token -1 in rows {np.flatnonzero(got.tokens < 0)}"
    compare(got, want, want_logits, configs, vocab, cap,
            label if want_cands else label + " (tokens only)")
    return got, want


def test_gumbel_k_vocab(sampler):
    wl = workloads.make("gumbel1024", 0, rows=48)
    got, _ = _check(sampler, wl.logits, wl.vocab, None, None, wl.configs, wl.uniforms, 64,
                    "gumbel k=V")
    assert ((got.flags & HS_ROW_LARGE) != 0).all()
    assert not (got.flags & HS_ROW_UNSUPPORTED).any()


def test_gumbel_full_batch_two_pass(sampler):
    """The 1024-row Gumbel workload at full size (k = vocab, top-p 0.98):
    every row through the two-pass kernel, tokens against the oracle."""
    wl = workloads.make("gumbel1024", 0)
    got, want = _check(sampler, wl.logits, wl.vocab, None, None, wl.configs, wl.uniforms, 64,
                       "gumbel 1024 x V", want_cands=False)
    two = (got.flags & HS_ROW_TWO_PASS) != 0
    print(f"[large] two-pass rows {int(two.sum())}/{two.size}; tokens equal "
          f"{int((got.tokens == want.token).sum())}, oracle draw margins < 1e-6: "
          f"{int((want.draw_margin < 1e-6).sum())}")
    assert two.mean() > 0.99


@pytest.mark.parametrize("name", ["gumbel", "normal", "low_t", "high_t", "penalised",
                                  "shifted_t02", "shifted_t01"])
def test_two_pass_distributions(sampler, name):
    """The two-pass kernel over other logit shapes and temperatures, with
    rows it must hand back (sorted ascending, so nearly every logit lies
    above the first chunk's maximum) mixed in.  The shifted cases put the
    maximum near 30 at T 0.2 and 0.1 (m0 / T of 150 to 300), where a
    per-row rounding of m0 / T shared by every bucket weight would move the
    bucket sums by more than the tolerated 1e-6."""
    rng = np.random.default_rng(len(name))
    rows, vocab = 40, 151936
    hist_ids = hist_off = None
    if name == "gumbel":
        logits = rng.gumbel(size=(rows, vocab)).astype(np.float32)
        cfg = dict(temperature=1.0, topK=float("inf"), topP=0.9)
    elif name == "normal":
        logits = (rng.standard_normal((rows, vocab)) * 2.5).astype(np.float32)
        cfg = dict(temperature=0.8, topK=float("inf"), topP=0.95)
    elif name == "low_t":
        logits = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
        cfg = dict(temperature=0.3, topK=vocab, topP=0.9)
    elif name == "high_t":
        logits = rng.gumbel(size=(rows, vocab)).astype(np.float32)
        cfg = dict(temperature=1.5, topK=float("inf"), topP=0.99)
    elif name == "shifted_t02":
        logits = (rng.standard_normal((rows, vocab)) * 2 + 20).astype(np.float32)
        cfg = dict(temperature=0.2, topK=float("inf"), topP=0.95)
    elif name == "shifted_t01":
        logits = (rng.gumbel(size=(rows, vocab)) + 20).astype(np.float32)
        cfg = dict(temperature=0.1, topK=float("inf"), topP=0.99)
    else:
        wl = workloads.make("v262k512", 4, rows=rows, vocab=vocab)
        logits, hist_ids, hist_off = wl.logits, wl.hist_ids, wl.hist_off
        cfg = dict(temperature=0.9, topK=float("inf"), topP=0.9, repetitionPenalty=1.15,
                   presencePenalty=0.4, frequencyPenalty=0.2)
    logits[3] = np.sort(logits[3])                 # handed back: rises past the first chunk
    logits[5, :1000] = -np.inf                     # a masked prefix
    u = rng.random(rows)
    u[7] = 0.0
    got, _ = _check(sampler, logits, vocab, hist_ids, hist_off, [cfg] * rows, u, 64,
                    f"two-pass {name}", want_cands=False)
    assert (got.flags[[r for r in range(rows) if r != 3]] & HS_ROW_TWO_PASS).all()
    assert not got.flags[3] & HS_ROW_TWO_PASS


@pytest.mark.parametrize("step", [1 / 64, 1 / 16])
def test_two_pass_block_walks(sampler, step):
    """Logits on a grid of `step` (N(0, 2.5^2), T 1, top-p 0.9): near the
    top-p crossing (v ~ 3) each grid value is held by about 180 (1/64) or 720
    (1/16) logits, so the located bucket's part holds more than 64 equal
    values (1/64) or the gathered list exceeds what one wave walks (1/16).
    Those walks take the whole workgroup's sort; draws near the top take the
    one-wave walk.  Tokens against the oracle."""
    rng = np.random.default_rng(int(1 / step))
    rows, vocab = 32, 151936
    logits = (np.round(rng.standard_normal((rows, vocab)) * 2.5 / step) * step).astype(np.float32)
    cfg = dict(temperature=1.0, topK=float("inf"), topP=0.9)
    u = rng.random(rows)
    got, _ = _check(sampler, logits, vocab, None, None, [cfg] * rows, u, 64,
                    f"two-pass grid {step}", want_cands=False)
    assert ((got.flags & HS_ROW_LARGE) != 0).all()


def test_partial_large_k(sampler):
    rng = np.random.default_rng(11)
    rows, vocab = 24, 151936
    logits = (rng.standard_normal((rows, vocab)) * 2.5).astype(np.float32)
    configs = [dict(temperature=float(rng.uniform(0.5, 1.5)), topK=int(rng.integers(1025, 9000)),
                    topP=float(rng.uniform(0.5, 0.995)), minP=0.0 if r % 3 else 0.01)
               for r in range(rows)]
    u = rng.random(rows)
    _check(sampler, logits, vocab, None, None, configs, u, 64, "partial large k")


def test_large_equal_logits(sampler):
    rows, vocab = 4, 20000
    logits = np.zeros((rows, vocab), np.float32)
    logits[1] = 1.5
    logits[2, ::7] = 2.0            # ties at two values
    logits[3, 100:130] = -np.inf    # excluded entries
    configs = [dict(temperature=1.0, topK=float("inf"), topP=0.5),
               dict(temperature=0.7, topK=0, topP=0.98),   # topK 0 -> 64: row kernel
               dict(temperature=1.0, topK=float("inf"), topP=0.9),
               dict(temperature=1.0, topK=5000.0, topP=0.95)]
    u = np.array([0.25, 0.5, 0.75, 0.999])
    _check(sampler, logits, vocab, None, None, configs, u, 64, "equal logits")
    _check(sampler, logits, vocab, None, None, configs, u, 64, "equal logits", want_cands=False)


def test_large_non_finite(sampler):
    rng = np.random.default_rng(5)
    rows, vocab = 4, 30000
    logits = (rng.standard_normal((rows, vocab)) * 2).astype(np.float32)
    logits[0, rng.choice(vocab, 500, replace=False)] = np.nan
    logits[1, rng.choice(vocab, 29990, replace=False)] = -np.inf   # 10 finite left
    logits[2, 17] = np.inf                                          # NaN probabilities
    logits[3, :] = np.nan
    logits[3, 9] = 1.0                                              # one candidate
    configs = [dict(temperature=1.0, topK=float("inf"), topP=0.9) for _ in range(rows)]
    u = np.array([0.3, 0.6, 0.9, 0.1])
    _check(sampler, logits, vocab, None, None, configs, u, 64, "non-finite")
    _check(sampler, logits, vocab, None, None, configs, u, 64, "non-finite", want_cands=False)


def test_large_with_penalties(sampler):
    wl = workloads.make("v262k512", 2, rows=8, vocab=60000)
    configs = [dict(c, topK=float("inf") if i % 2 else 3000) for i, c in enumerate(wl.configs)]
    configs[0] = dict(temperature=0.9, topK=2048, topP=0.9, repetitionPenalty=1.15)
    _check(sampler, wl.logits, wl.vocab, wl.hist_ids, wl.hist_off, configs, wl.uniforms, 64,
           "large k + penalties")
    _check(sampler, wl.logits, wl.vocab, wl.hist_ids, wl.hist_off, configs, wl.uniforms, 64,
           "large k + penalties", want_cands=False)


def test_min_p_and_top_p_edges_large(sampler):
    rng = np.random.default_rng(9)
    rows, vocab = 6, 40000
    logits = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    configs = [dict(temperature=1.0, topK=float("inf"), topP=0.0),
               dict(temperature=1.0, topK=float("inf"), topP=1.0),
               dict(temperature=1.0, topK=float("inf"), topP=0.9, minP=1.0),
               dict(temperature=1.0, topK=float("inf"), topP=0.9, minP=0.5),
               dict(temperature=0.05, topK=float("inf"), topP=0.99),
               dict(temperature=50.0, topK=float("inf"), topP=0.3)]
    u = np.array([0.5, 0.0, 0.7, 0.999999, 0.4, 0.2])
    _check(sampler, logits, vocab, None, None, configs, u, 64, "min-p / top-p edges")
    _check(sampler, logits, vocab, None, None, configs, u, 64, "min-p / top-p edges",
           want_cands=False)


HS_ROW_REPLAYED = 0x2


@pytest.mark.parametrize("k", [2048, 5000, 16384, 16385, 20000, 100000])
def test_large_k_ties_replayed(sampler, k):
    """Rows of many equal values with 1024 < k < the finite count: the order
    inside an equal-value group follows the reference's slot history
    (src/sampler.ts:55-74), which the slot replay reproduces (its slots in
    LDS up to k = 16384, in device memory above); tokens and candidate ids
    equal the oracle's, and no row is left unsupported."""
    rng = np.random.default_rng(k)
    rows = 12
    vocab = 60000 if k <= 16384 else 151936
    logits = np.round(rng.standard_normal((rows, vocab)) * 3).astype(np.float32)   # ~30 values
    logits[1] = np.round(logits[1] / 4)             # very coarse: a few huge groups
    logits[2, ::3] = np.nan
    configs = [dict(temperature=float(rng.uniform(0.5, 2.0)), topK=k, topP=float(rng.uniform(0.6, 1.0)))
               for _ in range(rows)]
    configs[3]["minP"] = 0.02
    u = rng.random(rows)
    u[4] = 0.0
    for want in (True, False):
        got, want_res = _check(sampler, logits, vocab, None, None, configs, u, 64,
                               f"ties k={k}", want_cands=want)
        assert (got.flags & HS_ROW_REPLAYED).any()


def test_large_k_ties_beyond_2_19(sampler):
    """Top-k above 2^19 on a 600000-logit vocabulary of coarse values (a few
    dozen distinct ones): the device-memory replay's four-level min tree,
    tokens and candidate ids equal to the oracle's."""
    rng = np.random.default_rng(11)
    rows, vocab = 2, 600000
    logits = np.round(rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    configs = [dict(temperature=1.0, topK=550000, topP=0.9),
               dict(temperature=0.7, topK=530000, topP=0.99)]
    u = np.array([0.999, 0.31])
    for want in (True, False):
        got, _ = _check(sampler, logits, vocab, None, None, configs, u, 64,
                        "ties k > 2^19", want_cands=want)
        assert (got.flags & HS_ROW_REPLAYED).all()


@pytest.mark.parametrize("k,cap", [(5000, 2000), (30000, 1500)])
def test_large_k_ties_long_candidate_lists(sampler, k, cap):
    """More candidate positions with ties than the LDS replay orders (1024):
    the device-memory replay orders them (value descending, slot ascending,
    src/sampler.ts:72-75); ids, probabilities and tokens equal the oracle's."""
    rng = np.random.default_rng(k + cap)
    rows, vocab = 6, 151936
    logits = (np.round(rng.standard_normal((rows, vocab)) * 8) / 4).astype(np.float32)
    configs = [dict(temperature=1.0, topK=k, topP=0.999) for _ in range(rows)]
    u = rng.random(rows)
    got, _ = _check(sampler, logits, vocab, None, None, configs, u, cap, f"ties k={k} cap={cap}")
    assert (got.flags & HS_ROW_REPLAYED).all()
