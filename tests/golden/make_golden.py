"""Write the golden fixtures of the verify path with the oracle.

Each fixture holds seeded inputs and the oracle's outputs for one part of
the path, sized to stay small:
  qgemm.npz     Q4_K / Q6_K / Q8_0 weights (GGUF block bytes), x [5][k], y
  attn.npz      the 16-node draft tree over an f16 cache, scale 1/sqrt(d)
  sampler.npz   logits rows and their distributions under four settings
  accept.npz    acceptance rounds (greedy, rejection with and without draft
                logits, gumbel) with explicit uniforms
  stream.npz    a micro model's free-running greedy speculative stream

    python tests/golden/make_golden.py      # rewrites tests/golden/*.npz
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.dirname(HERE)):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import cpvo  # noqa: E402

import model_fixtures as mf  # noqa: E402

TREE16 = np.array([-1, -1, -1, -1, 0, 0, 0, 1, 1, 1, 4, 4, 4, 10, 10, 10], dtype=np.int32)

SAMPLER_SETTINGS = [  # (temp, top_k, top_p, min_p, min_keep, repeat, freq, present, last_n)
    (0.7, 0, 0.95, 0.0, 1, 1.0, 0.0, 0.0, 64),
    (1.0, 0, 1.0, 0.0, 1, 1.0, 0.0, 0.0, 64),
    (0.8, 40, 0.9, 0.05, 1, 1.0, 0.0, 0.0, 64),
    (0.9, 0, 1.0, 0.02, 1, 1.3, 0.1, 0.2, 16),
]

MICRO = dict(mf.TINY, n_layer=2, n_embd=256, n_head=4, n_head_kv=1, head_dim=64, n_ff=512, n_vocab=2048)
MICRO_SEED, MICRO_PROMPT, MICRO_GEN, MICRO_DEPTH = 5, 40, 24, 3


def params(row):
    return cpvo.SamplerParams(*[float(v) if i in (0, 2, 3, 5, 6, 7) else int(v) for i, v in enumerate(row)])


def make_qgemm(rng):
    out = {}
    for name, t, n, k in (("q4_k", cpvo.Q4_K, 32, 512), ("q6_k", cpvo.Q6_K, 32, 512), ("q8_0", cpvo.Q8_0, 32, 256)):
        wq = cpvo.quantize(t, rng.normal(0, 0.02, size=(n, k)).astype(np.float32))
        x = rng.normal(0, 1, size=(5, k)).astype(np.float32)
        out[f"{name}_w"] = wq
        out[f"{name}_x"] = x
        out[f"{name}_y"] = cpvo.qgemm(t, wq, x)
        out[f"{name}_shape"] = np.array([t, n, k], dtype=np.int64)
    return out


def make_attn(rng):
    n_past, t, h, hkv, d = 100, 16, 2, 1, 64
    k = cpvo.f32_to_f16_bits(rng.normal(size=(n_past + t, hkv * d)).astype(np.float32))
    v = cpvo.f32_to_f16_bits(rng.normal(size=(n_past + t, hkv * d)).astype(np.float32))
    q = rng.normal(size=(t, h, d)).astype(np.float32)
    scale = np.float32(1) / np.sqrt(np.float32(d))
    out = cpvo.attn(q, k, v, n_past, TREE16.tolist(), scale)
    return dict(q=q, k=k, v=v, parent=TREE16, dims=np.array([n_past, t, h, hkv, d], dtype=np.int64),
                scale=np.array([scale], dtype=np.float32), out=out)


def make_sampler(rng):
    V, rows = 1000, 4
    logits = rng.normal(0, 3, size=(rows, V)).astype(np.float32)
    logits[np.arange(rows), rng.integers(V, size=rows)] += 8
    hist = rng.integers(0, 50, size=(rows, 24)).astype(np.int32)
    hist[:, :3] = -1
    out = dict(logits=logits, hist=hist, settings=np.array(SAMPLER_SETTINGS, dtype=np.float64))
    for si, row in enumerate(SAMPLER_SETTINGS):
        p = params(row)
        ids = np.full((rows, V), -1, dtype=np.int32)
        probs = np.zeros((rows, V), dtype=np.float32)
        n = np.zeros(rows, dtype=np.int32)
        for r in range(rows):
            h = [x for x in hist[r] if x >= 0][-p.penalty_last_n:]
            i, pr, _ = cpvo.distribution(p, logits[r], h)
            n[r] = i.size
            ids[r, :i.size] = i
            probs[r, :i.size] = pr
        out[f"s{si}_ids"], out[f"s{si}_probs"], out[f"s{si}_n"] = ids, probs, n
    return out


def make_accept(rng):
    B, k, V = 4, 4, 500
    pl = rng.normal(0, 1.5, size=(B, k + 1, V)).astype(np.float32)
    pl[:, :, 7] += 9
    q = (pl[:, :k] + rng.normal(0, 1, size=(B, k, V))).astype(np.float32)
    draft = pl[:, :k].argmax(axis=2).astype(np.int32)
    draft[1, 1] = 3
    draft[3, 0] = 11
    u = rng.random(size=(B, k + 1, 2)).astype(np.float32)
    T = np.float32(0.7)
    uu = rng.random(size=(B, k + 1, V)).astype(np.float32)
    noise = ((-np.log(-np.log(np.maximum(uu, 1e-12)))) * T).astype(np.float32)
    pr = params(SAMPLER_SETTINGS[0])
    out = dict(p_logits=pl, q_logits=q, draft=draft, u=u, noise=noise)
    cases = {
        "greedy": (cpvo.SamplerParams(), cpvo.ACCEPT_GREEDY, {}),
        "reject": (pr, cpvo.ACCEPT_REJECT, dict(u=u)),
        "reject_q": (pr, cpvo.ACCEPT_REJECT, dict(u=u, q_logits=q)),
        "gumbel_plain": (cpvo.SamplerParams(temp=0.7), cpvo.ACCEPT_GUMBEL, dict(noise_t=noise)),
        "gumbel_top_p": (pr, cpvo.ACCEPT_GUMBEL, dict(noise_t=noise)),
    }
    for name, (p, mode, kw) in cases.items():
        tok, n = cpvo.spec_accept(pl, draft, p, mode, **kw)
        out[f"{name}_tok"], out[f"{name}_n"] = tok, n
    return out


def micro_prompt():
    return np.random.default_rng(MICRO_SEED + 1).integers(0, MICRO["n_vocab"], size=MICRO_PROMPT).tolist()


def make_stream():
    m = cpvo.Model(MICRO)
    mf.load_into(m, mf.make_tensors(MICRO, seed=MICRO_SEED))
    s = cpvo.Session(m, 256)
    toks, st = s.fused_generate(micro_prompt(), MICRO_GEN, MICRO_DEPTH, tail=16, bulk=32)
    s.free()
    m.free()
    return dict(tokens=np.array(toks, dtype=np.int32), stats=np.array(st, dtype=np.int64))


MAKERS = {"qgemm": make_qgemm, "attn": make_attn, "sampler": make_sampler, "accept": make_accept,
          "stream": lambda rng: make_stream()}


def build(name):
    return MAKERS[name](np.random.default_rng(20260 + list(MAKERS).index(name)))


def main():
    for name in MAKERS:
        data = build(name)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
