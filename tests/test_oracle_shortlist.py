"""The shortlist draft head's index quirk, decided on the oracle.

With a shortlist (MtpTail::n_cand), each link's draft is cands[argmax]
(qwen35.rs:1904-1910), but the graph feeds the argmax itself, the index
into the shortlist, to the next link's embedding (tok_src = ids, :2958).
The same candidate set in identity order (0..n-1, where index and token
coincide) and in a permuted order therefore gives the same first-link
drafts, while the second link embeds different tokens and differs.  Were
the token fed instead, both orders would give the same chain.
"""
import numpy as np

from oracle import cpvo

import model_fixtures as mf

SMALL = dict(mf.TINY, n_layer=2, n_vocab=4096)


def test_next_link_embeds_the_shortlist_index():
    m = cpvo.Model(SMALL)
    mf.load_into(m, mf.make_tensors(SMALL, seed=3))
    n = 512
    ident = list(range(n))
    perm = np.random.default_rng(5).permutation(n).tolist()
    prompt = np.random.default_rng(6).integers(0, SMALL["n_vocab"], size=30).tolist()
    chains = []
    for cands in (ident, perm):
        s = cpvo.Session(m, 64)
        s.prefill(prompt[:25])
        P, C, CF, _, _ = s.step_fused_cached(prompt[25:], 2, cands=cands)
        chains.append((P, C, CF))
        s.free()
    (P0, C0, F0), (P1, C1, F1) = chains
    assert np.array_equal(P0, P1)
    assert np.array_equal(C0[0], C1[0])            # link 0: the same tokens
    assert np.array_equal(F0[0], F1[0])
    assert not np.array_equal(C0[1], C1[1]) or not np.array_equal(F0[1], F1[1])   # link 1 differs
    m.free()
