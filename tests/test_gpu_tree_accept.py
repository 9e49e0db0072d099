"""GPU tree acceptance (sh_tree_accept) vs the oracle (or_tree_accept) on
configs[3]-shaped trees: depth 3 with branching 4, 3, 2 (1 + 4 + 12 + 24 = 41
nodes), target logits N(0, 3), draft logits = target + N(0, 1) at every node,
children drawn from the draft distribution at T = 1 (inverse CDF with the
oracle's Philox stream). Paths and next tokens must be identical for Philox
uniforms (shared seed), explicit uniforms and greedy."""
import numpy as np
import pytest

import oracle as O
from seeker_amd import SeekerError
from seeker_amd import synth as S
from seeker_amd._native import SH_ERR_ARG, SH_SAMPLE_GREEDY, SH_SAMPLE_REJECTION, sh_sampling

pytestmark = pytest.mark.gpu


def tree_parents(branching):
    parents, level = [-1], [0]
    for b in branching:
        nxt = []
        for v in level:
            for _ in range(b):
                parents.append(v)
                nxt.append(len(parents) - 1)
        level = nxt
    return np.array(parents, dtype=np.int32)


def make_trees(B, V, branching, seed=11, T=1.0):
    par = tree_parents(branching)
    n = par.size
    p = S.normal_f32(seed, 20, B * n * V, 0.0, 3.0).reshape(B, n, V)
    q = (p + S.normal_f32(seed, 21, B * n * V, 0.0, 1.0).reshape(B, n, V)).astype(np.float32)
    u = O.philox_uniforms(seed, 22, 0, B * n)
    tokens = np.zeros((B, n), dtype=np.uint32)
    for b in range(B):
        tokens[b, 0] = b  # the root's token is not read
        for c in range(1, n):
            tokens[b, c] = O.sample_vocab_order(q[b, par[c]], T, float(u[b * n + c]))
    return p, q, tokens, np.tile(par, (B, 1))


def run_gpu(engine, p, q, tokens, parents, mode, T, seed, uniforms=None):
    B, n, V = p.shape
    bufs = [engine.to_device(x) for x in (p, q, tokens, parents)]
    path, plen, nxt = engine.dev_alloc(4 * B * n), engine.dev_alloc(4 * B), engine.dev_alloc(4 * B)
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = mode, T, seed, 0
    keep = None
    if uniforms is not None:
        keep = np.ascontiguousarray(uniforms, np.float32)
        s.uniforms = keep.ctypes.data_as(O.F32P)
    engine.tree_accept(bufs[0], bufs[1] if mode == SH_SAMPLE_REJECTION else None, bufs[2], bufs[3], B, n, V, s,
                       path, plen, nxt)
    pa = path.read(np.uint32, B * n).reshape(B, n)
    pl, nt = plen.read(np.uint32, B), nxt.read(np.uint32, B)
    for x in bufs + [path, plen, nxt]:
        x.free()
    return [pa[b, : pl[b]].tolist() for b in range(B)], nt


def oracle_uniforms(seed, B, n):
    return O.philox_uniforms(seed, 0x5EC, 0, 2 * B * n).reshape(B, n, 2)


@pytest.mark.parametrize("B,V", [(4, 1000), (4, 128256)])
def test_tree_rejection_matches_oracle(engine, B, V):
    print(f"tree rejection B={B} V={V}", flush=True)
    p, q, tokens, parents = make_trees(B, V, (4, 3, 2))
    paths, nt = run_gpu(engine, p, q, tokens, parents, SH_SAMPLE_REJECTION, 1.0, seed=11)
    U = oracle_uniforms(11, B, parents.shape[1])
    for b in range(B):
        opath, onext = O.tree_accept(p[b], q[b], tokens[b], parents[b], 1.0, U[b])
        print(f"  tree {b}: path {paths[b]} next {nt[b]}", flush=True)
        assert paths[b] == opath and nt[b] == onext, b


def test_tree_explicit_uniforms_and_lengths(engine):
    """Explicit uniforms spanning accept-everything (u = 0) to reject-everything
    (u ~ 1): the full-depth path and the root resample both occur."""
    B, V = 6, 500
    p, q, tokens, parents = make_trees(B, V, (4, 3, 2), seed=5)
    n = parents.shape[1]
    U = np.random.default_rng(3).random((B, n, 2)).astype(np.float32)
    U[0, :, 0] = 0.0            # every first child accepted: path to a leaf
    U[1, :, 0] = 0.99999994     # rejections everywhere likely
    paths, nt = run_gpu(engine, p, q, tokens, parents, SH_SAMPLE_REJECTION, 1.0, seed=0, uniforms=U)
    for b in range(B):
        opath, onext = O.tree_accept(p[b], q[b], tokens[b], parents[b], 1.0, U[b])
        assert paths[b] == opath and nt[b] == onext, b
    assert len(paths[0]) == 4  # root + one node per level


def test_tree_greedy(engine):
    B, V = 4, 300
    p, q, tokens, parents = make_trees(B, V, (4, 3, 2), seed=9)
    # make some greedy paths long: child 1 of each node carries the argmax of its parent
    n = parents.shape[1]
    for b in range(B):
        for c in range(1, n):
            if c == min(i for i in range(1, n) if parents[b, i] == parents[b, c]):
                tokens[b, c] = int(np.argmax(p[b, parents[b, c]])) if b % 2 == 0 else tokens[b, c]
    paths, nt = run_gpu(engine, p, None, tokens, parents, SH_SAMPLE_GREEDY, 0.0, seed=0)
    for b in range(B):
        opath, onext = O.tree_accept(p[b], p[b], tokens[b], parents[b], 0.0, np.zeros((n, 2), np.float32))
        assert paths[b] == opath and nt[b] == onext, b
    assert len(paths[0]) == 4 and len(paths[2]) == 4


def test_tree_malformed_rejected(engine):
    B, V = 1, 50
    p, q, tokens, parents = make_trees(B, V, (2, 2), seed=1)
    bad = parents.copy()
    bad[0, 3] = 5
    with pytest.raises(SeekerError) as e:
        run_gpu(engine, p, q, tokens, bad, SH_SAMPLE_REJECTION, 1.0, seed=1)
    assert e.value.status == SH_ERR_ARG


def test_greedy_argmax_special_values(engine):
    """Greedy argmax on rows with NaN, +-inf and ties, through the greedy tree
    walk (the same device key, sh_amax_key, as k_argmax): the host rule of
    inference/sample.rs:504-514 as or_argmax states it (the first x[i] > best,
    best from -inf): NaN and -inf never win, a row without a value above -inf
    gives 0, ties give the lowest index. Each tree's root row is one case; its
    first child carries the root's expected argmax, so the walk accepts it and
    the next token is the child row's argmax (a second case)."""
    print("greedy argmax special values", flush=True)
    V, nan, inf = 300, np.float32(np.nan), np.float32(np.inf)
    rng = np.random.default_rng(5)
    rows = []
    r = rng.standard_normal(V).astype(np.float32); r[rng.integers(0, V, 40)] = nan; rows.append(r)  # NaNs sprinkled
    rows.append(np.full(V, nan, np.float32))                                                          # all NaN
    rows.append(np.full(V, -inf, np.float32))                                                         # all -inf
    r = np.full(V, -inf, np.float32); r[0] = nan; rows.append(r)                                      # NaN, then -inf
    r = np.full(V, -inf, np.float32); r[150] = r[200] = 5.0; rows.append(r)                           # tie
    r = rng.standard_normal(V).astype(np.float32); r[77] = r[99] = inf; rows.append(r)                # +inf tie
    r = np.full(V, nan, np.float32); r[3] = inf; rows.append(r)                                       # NaN, +inf
    r = np.full(V, -inf, np.float32); r[5] = np.float32(-3e38); rows.append(r)                        # lowest finite
    r = np.full(V, nan, np.float32); r[290] = -1.0; r[10] = -1.0; rows.append(r)                      # tie among NaN
    r = rng.standard_normal(V).astype(np.float32); r[::2] = -inf; rows.append(r)                      # half -inf
    B, n = len(rows) // 2, 3
    par = np.array([-1, 0, 0], np.int32)
    p = np.zeros((B, n, V), np.float32)
    tokens = np.zeros((B, n), np.uint32)
    for b in range(B):
        p[b, 0], p[b, 1] = rows[2 * b], rows[2 * b + 1]
        p[b, 2] = rng.standard_normal(V).astype(np.float32)
        tokens[b, 1] = O.argmax(p[b, 0])
        tokens[b, 2] = (O.argmax(p[b, 0]) + 1) % V
    q = np.zeros_like(p)
    parents = np.tile(par, (B, 1))
    paths, nxt = run_gpu(engine, p, q, tokens, parents, SH_SAMPLE_GREEDY, 0.0, 0)
    for b in range(B):
        want_path, want_next = O.tree_accept(p[b], q[b], tokens[b], par, 0.0, np.zeros((n, 2), np.float32))
        assert want_path == [0, 1], (b, want_path)
        assert (paths[b], int(nxt[b])) == (want_path, want_next), (b, paths[b], int(nxt[b]), want_next)
    # the oracle's rule itself on the cases above
    assert [O.argmax(x) for x in rows[1:9]] == [0, 0, 0, 150, 77, 3, 5, 10]
