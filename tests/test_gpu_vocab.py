"""GPU vocabulary scoring, top-k and the next-token pick (model.rs:2842-2907,
cuda.rs:3052-3111, kernels.rs:1085-1228) against the oracle's
orc_vocab_select: tokens, scores and ids bit-identical, at the 256000-token
vocabulary of the bench model and on the reference's own top-k test vector.
"""

from __future__ import annotations

import numpy as np
import pytest

from test_gpu_decode import TINY, THREADS, assert_same_tokens

pytestmark = pytest.mark.gpu

V = 256000


def logits_case(seed: int, vocab: int, ties: bool):
    rng = np.random.default_rng(seed)
    if ties:  # few distinct values: equal scores everywhere, ids break the ties
        lg = (rng.integers(-300, 300, vocab) * 0.03125).astype(np.float32)
    else:
        lg = (rng.standard_normal(vocab) * 6.0).astype(np.float32)
    lg[rng.integers(0, vocab, 5)] = np.nan
    lg[[1, 2, 105, 106]] = 40.0  # the early ids: masked while fewer than 4 tokens were generated
    valid = (rng.random(vocab) > 0.05).astype(np.uint8)
    top = np.argsort(-np.nan_to_num(lg, nan=-1e30), kind="stable")[:12]
    recent = np.concatenate([top[:6], top[:3], rng.integers(0, vocab, 20)])[:32].astype(np.int32)
    return lg, valid, recent


def check_select(backend, dev, orc, d_lg, d_valid, d_recent, lg, valid, recent, scoring, gen, temp, pos, k, what):
    tok = backend.HipBuffer.from_host(dev, np.array([-7], np.int32))
    sc = backend.HipBuffer.alloc(dev, k)
    ids = backend.HipBuffer.alloc(dev, k, np.int32)
    dev.vocab_select(d_lg, lg.size, d_valid, d_recent, len(recent), gen, scoring, temp, pos, k, tok, sc, ids)
    dev.sync()
    want_tok, want_sc, want_ids = orc.vocab_select(lg, valid, recent, gen, scoring, temp, pos, k)
    n = want_ids.size
    got_sc, got_ids = sc.numpy(), ids.numpy()
    assert int(tok.numpy()[0]) == want_tok, what
    assert np.array_equal(got_ids[:n], want_ids), what
    assert np.array_equal(got_sc[:n].view(np.uint32), want_sc.view(np.uint32)), what
    assert np.all(got_ids[n:] == -1) and np.all(got_sc[n:] == -np.inf), what


@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("scoring", [0, 1])
def test_vocab_select_256k_bit_exact(backend, dev, orc, scoring, ties):
    lg, valid, recent = logits_case(50 + scoring + 2 * ties, V, ties)
    print(f"\n[vocab_select] V={V} scoring={scoring} ties={ties}", flush=True)
    d_lg = backend.HipBuffer.from_host(dev, lg)
    d_valid = backend.HipBuffer.from_host(dev, valid)
    d_recent = backend.HipBuffer.from_host(dev, recent)
    cases = [(0, 0.0, 1, 7), (9, 0.0, 40, 100), (3, 0.0, 64, 1), (9, 0.8, 40, 517), (3, 1.5, 64, 12345),
             (9, 0.05, 40, 99), (9, 30.0, 40, 4242)]
    cases += [(9, 1.0, 40, p) for p in range(200, 216)]
    for gen, temp, k, pos in cases:
        check_select(backend, dev, orc, d_lg, d_valid, d_recent, lg, valid, recent, scoring, gen, temp, pos, k,
                     f"gen={gen} t={temp} k={k} pos={pos}")
    # no mask, no recent ids
    check_select(backend, dev, orc, d_lg, None, None, lg, None, np.zeros(0, np.int32), scoring, 9, 0.7, 3, 40,
                 "unmasked")


def test_vocab_select_edges(backend, dev, orc):
    # fewer candidates than k, no candidate at all (token 506), one-element vocabularies
    for vocab, valid_frac, k in ((100, 0.3, 40), (50, 0.0, 8), (1, 1.0, 1), (2049, 1.0, 64), (4096, 0.01, 64)):
        rng = np.random.default_rng(vocab)
        lg = rng.standard_normal(vocab).astype(np.float32)
        valid = (rng.random(vocab) < valid_frac).astype(np.uint8)
        recent = rng.integers(0, vocab, 5).astype(np.int32)
        d_lg = backend.HipBuffer.from_host(dev, lg)
        d_valid = backend.HipBuffer.from_host(dev, valid)
        d_recent = backend.HipBuffer.from_host(dev, recent)
        for scoring in (0, 1):
            for temp in (0.0, 0.9):
                check_select(backend, dev, orc, d_lg, d_valid, d_recent, lg, valid, recent, scoring, 9, temp, 11, k,
                             f"vocab={vocab} scoring={scoring} t={temp}")


def partition_bounds(vocab: int, parts: int, p: int):
    return vocab * p // parts, vocab * (p + 1) // parts


def check_topk(backend, dev, orc, lg, valid, recent, gen, k, parts, sample=None):
    vocab = lg.size
    d_lg = backend.HipBuffer.from_host(dev, lg)
    d_valid = backend.HipBuffer.from_host(dev, valid)
    d_recent = backend.HipBuffer.from_host(dev, np.asarray(recent, np.int32))
    sc = backend.HipBuffer.alloc(dev, parts * k)
    ids = backend.HipBuffer.alloc(dev, parts * k, np.int32)
    dev.vocab_topk(d_lg, d_valid, d_recent, sc, ids, vocab, len(recent), gen, k, parts)
    dev.sync()
    got_sc, got_ids = sc.numpy().reshape(parts, k), ids.numpy().reshape(parts, k)
    for p in (range(parts) if sample is None else sample):
        a, b = partition_bounds(vocab, parts, p)
        vp = np.zeros(vocab, np.uint8)
        vp[a:b] = valid[a:b]
        _, want_sc, want_ids = orc.vocab_select(lg, vp, recent, gen, 1, 0.0, 0, k)
        n = want_ids.size
        assert np.array_equal(got_ids[p, :n], want_ids), (parts, p)
        assert np.array_equal(got_sc[p, :n].view(np.uint32), want_sc.view(np.uint32)), (parts, p)
        assert np.all(got_ids[p, n:] == -1) and np.all(got_sc[p, n:] == -np.inf), (parts, p)
    return got_sc, got_ids


def test_vocab_topk_reference_known_answer(backend, dev, orc):
    """ops_test.rs:165-212: the partitions' candidates hold the exact global
    top-40 of the penalised logits."""
    N, K, P = 4096, 40, 8
    i = np.arange(N)
    logits = (((i * 7919) % 65521).astype(np.float32) * np.float32(0.001) +
              i.astype(np.float32) * np.float32(1e-7)).astype(np.float32)
    valid = (i % 17 != 0).astype(np.uint8)
    recent = [31, 777, 2049, 4001]
    sc, ids = check_topk(backend, dev, orc, logits, valid, recent, 10, K, P)
    cand = sorted(zip(sc.ravel().tolist(), ids.ravel().tolist()), key=lambda e: (-e[0], e[1]))[:K]
    expected = sorted(((float(logits[t] - np.float32(1.8)) if t in recent else float(logits[t]), t)
                       for t in range(N) if valid[t]), key=lambda e: (-e[0], e[1]))[:K]
    assert cand == expected


@pytest.mark.parametrize("parts,k", [(128, 40), (128, 1), (1, 40), (7, 64), (3000, 5)])
def test_vocab_topk_256k_partitions(backend, dev, orc, parts, k):
    """Partitions of 2000 ids (the reference's 128), and partitions larger
    than one workgroup's 2048 ids (the reference's generic kernel), against
    the oracle per partition."""
    lg, valid, recent = logits_case(70 + parts, V, ties=True)
    print(f"\n[vocab_topk] V={V} partitions={parts} k={k}", flush=True)
    sample = None if parts <= 8 else list(range(0, parts, max(1, parts // 12))) + [parts - 1]
    sc, ids = check_topk(backend, dev, orc, lg, valid, list(recent), 2, k, parts, sample)
    # the union of the partitions holds the global best k (model.rs:2801-2870)
    flat = [(s, t) for s, t in zip(sc.ravel().tolist(), ids.ravel().tolist()) if t >= 0]
    flat.sort(key=lambda e: (-e[0], e[1]))
    _, want_sc, want_ids = orc.vocab_select(lg, valid, list(recent), 2, 1, 0.0, 0, k)
    assert [t for _, t in flat[:k]] == want_ids.tolist()


def test_vocab_rejects_bad_arguments(backend, dev):
    lg = backend.HipBuffer.alloc(dev, 100)
    tok = backend.HipBuffer.alloc(dev, 1, np.int32)
    with pytest.raises(backend.HipError):
        dev.vocab_select(lg, 100, k=65, token=tok)
    with pytest.raises(backend.HipError):
        dev.vocab_select(lg, 100, scoring=2, token=tok)
    with pytest.raises(backend.HipError):
        dev.vocab_select(lg, 100, n_recent=3, token=tok)  # recent ids missing
    with pytest.raises(backend.HipError):
        dev.vocab_topk(lg, None, None, lg, tok, 100, 0, 9, 1, 101)  # more partitions than ids


# ---------------------------------------------------------------- the token step's pick

def oracle_sampled_decode(orc, model, prompt, n_decode, valid, temperature, top_k):
    """step_generation's loop (model.rs:2713-2930) over the oracle's token step:
    teacher-forced through the prompt, then the pick of the CPU path."""
    o = orc.OracleGemma2(model)
    P, total = len(prompt), len(prompt) + n_decode
    lg = np.zeros(model["cfg"]["vocab"], np.float32)
    picks, history = [], []
    tok = int(prompt[0])
    for pos in range(total):
        o.step(tok, pos, threads=THREADS, logits=lg)
        history.append(tok)
        gen = max(0, pos - (P - 1))
        k = top_k if temperature > 0 else 1
        nxt = orc.vocab_select(lg, valid, history[-32:], gen, 0, temperature, pos + 1, k)[0]
        picks.append(nxt)
        tok = int(prompt[pos + 1]) if pos + 1 < P else nxt
    return np.array(picks, np.int32)


@pytest.mark.parametrize("temperature", [0.0, 0.9])
def test_gemma2_step_sampler_matches_oracle(backend, dev, orc, synth, temperature):
    """The step with a sampler (masks, softcap, recent-token penalty, the
    draw) picks the oracle's tokens at every position, captured in one graph."""
    model = synth.gemma2_model(TINY, seed=21)
    prompt = synth.prompt_tokens(6, TINY["vocab"], seed=4)
    n_dec = 40
    rng = np.random.default_rng(5)
    valid = (rng.random(TINY["vocab"]) > 0.2).astype(np.uint8)
    m = backend.Gemma2Model.from_host(dev, model)
    d_valid = backend.HipBuffer.from_host(dev, valid)
    m.set_sampler(temperature=temperature, top_k=40, valid=d_valid)
    total = len(prompt) + n_dec
    state = backend.HipBuffer.from_host(dev, np.array([prompt[0], 0], np.int32))
    hist = backend.HipBuffer.from_host(dev, np.full(total, -1, np.int32))
    pr = backend.HipBuffer.from_host(dev, np.asarray(prompt, np.int32))
    kc = backend.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    vc = backend.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    graph = dev.capture(lambda: m.step(state, kc, vc, hist=hist, hist_cap=total, prompt=pr,
                                       prompt_len=len(prompt)))
    for _ in range(total):
        graph.launch()
    dev.sync()
    got = hist.numpy()
    graph.close()
    m.close()
    want = oracle_sampled_decode(orc, model, prompt, n_dec, valid, temperature, 40)
    assert_same_tokens(got, want)
    # the penalty is live: the plain argmax decode differs somewhere
    o = orc.OracleGemma2(model)
    greedy, tok = [], int(prompt[0])
    lg = np.zeros(TINY["vocab"], np.float32)
    for pos in range(total):
        nxt = o.step(tok, pos, threads=THREADS, logits=lg)
        greedy.append(nxt)
        tok = int(prompt[pos + 1]) if pos + 1 < len(prompt) else nxt
    assert not np.array_equal(np.array(greedy, np.int32), want)


def test_gemma2_prefill_sampler_then_steps(backend, dev, orc, synth):
    """A batched prefill records the prompt's tokens for the penalty and picks
    with no token generated; the steps that follow continue the oracle's
    sampled sequence."""
    cfg = dict(TINY, ctx_len=128)
    model = synth.gemma2_model(cfg, seed=22)
    prompt = synth.prompt_tokens(45, cfg["vocab"], seed=9)
    n_dec = 20
    temperature = 0.9
    m = backend.Gemma2Model.from_host(dev, model)
    m.set_sampler(temperature=temperature, top_k=40)
    P, total = len(prompt), len(prompt) + n_dec
    kc = backend.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    vc = backend.HipBuffer.from_host(dev, np.zeros(m.cache_elems(), np.uint16))
    am = backend.HipBuffer.from_host(dev, np.array([-1], np.int32))
    toks = backend.HipBuffer.from_host(dev, np.asarray(prompt, np.int32))
    m.prefill(toks.ptr, 30, 0, kc, vc)
    m.prefill(toks.ptr + 4 * 30, P - 30, 30, kc, vc, argmax=am)
    dev.sync()
    first = int(am.numpy()[0])
    state = backend.HipBuffer.from_host(dev, np.array([first, P], np.int32))
    hist = backend.HipBuffer.from_host(dev, np.full(total, -1, np.int32))
    for _ in range(n_dec):
        m.step(state, kc, vc, hist=hist, hist_cap=total, prompt_len=P)
    dev.sync()
    got = hist.numpy()
    m.close()
    want = oracle_sampled_decode(orc, model, prompt, n_dec, None, temperature, 40)
    assert first == want[P - 1]
    assert_same_tokens(got[P:], want[P:])
