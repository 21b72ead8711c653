#!/usr/bin/env python3
"""Verify-step latency and accepted tokens/s: 27B-class Q4_K model, draft k=4, one MI355X.

Workload: the end-to-end 27B-class configuration -- 64 layers, d_model 5120,
40 Q / 8 KV heads x 128, SwiGLU FFN 17408, vocab 151,936, qwen35 layout (attn_q
packs Q and the per-head output gate, q/k norms), every linear weight Q4_K,
token embedding and output head Q6_K, norms 1, one MTP (nextn) layer; random
weights generated on the device (no checkpoint); a 4096-token uniform random
prompt; context 32768; greedy speculative decoding with k=4 drafts from the
4-link MTP chain.

A step is one round of the fused loop (crates/codpiece-cli/src/main.rs:
803-913): [last] + 4 drafts through the trunk, the LM head argmax, the MTP
chain, greedy acceptance and the KV rewind.  `value` is committed tokens per
second over the timed rounds (host loop included); `ms_per_step` the wall
time of a round.  With random weights the drafts are almost never accepted,
so a round commits ~1 token, as the reference would on the same weights.

Beside the line's required fields, `detail` holds:
  * the device time of a round and of a verify-only round (depth 0), of a
    round with the 8192-token shortlist head, and of the 16-node tree verify
    and its branch commit, from HIP events on the library's stream;
  * kernel_classes: extra rounds run with cpv_profile_start/stop, which
    records every GEMM and attention launch; cpv_profile_replay launches
    each class's recorded launches again back to back between one pair of
    HIP events on the library's stream (per-launch events would add the
    dispatch gaps); `roofline.achieved` = the dominant class's mean
    algorithmic bytes per launch / its mean replayed launch time;
  * step_cost_us: verify-only device time at T = 1, 2, 4, 8, 16 tokens
    (main.rs:549-629);
  * oracle_drafts: the fused loop with drafts from the plain greedy stream
    (acceptance 1.0), accepted tok/s when every draft is right;
  * greedy_run and sampled_T0.7_top_p0.95: the workload's two full runs,
    512 new tokens each (greedy, and T = 0.7 / top-p 0.95 with the engine's
    post-commit re-draft), from a fresh prefill;
  * gemm: the Q4_K and Q8_0 GEMMs at the four verify shapes x M in
    {1, 5, 8, 16}, weights rotated over >= 512 MB;
  * attention_tree16: tree attention at context 8192 and 32768;
  * acceptance_sampler: the acceptance sampler at B = 1, 4, 16;
  * prefill: the prompt's prefill and its wide GEMM.
`cpu_baseline` runs whole verify rounds of the oracle (the C restatement of
the reference's CPU path under oracle/) on the host threads this process is
given, median of 5 -- a reported baseline, not the target; cpu_configs times
the oracle's functions at the microbench shapes.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HP = dict(n_layer=64, n_embd=5120, n_head=40, n_head_kv=8, head_dim=128, n_ff=17408, n_vocab=151936,
          n_rot=128, rope_sections=(22, 22, 20, 0), rms_eps=1e-6, freq_base=1e6, has_mtp=True)
HBM_PEAK_GBS = 8000.0
# the verify GEMM shapes (k, n): q|k|v of the gateless layout, wo, gate (= up), down
GEMM_SHAPES = ((5120, 7168), (5120, 5120), (5120, 17408), (17408, 5120))
# the canonical 16-node draft tree (widths 4, 6, 3, 3)
TREE16 = [-1, -1, -1, -1, 0, 0, 0, 1, 1, 1, 4, 4, 4, 10, 10, 10]
INT8_MFMA_PEAK_TOPS = 5000.0   # dense int8 MFMA, TOP/s
Q8_0, Q4_K, Q6_K, F32 = 8, 12, 14, 0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=16, help="timed rounds")
    ap.add_argument("--warmup", type=int, default=3, help="untimed rounds before the timed ones")
    ap.add_argument("--layers", type=int, default=HP["n_layer"], help="trunk layers (64 = the workload)")
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--prefill-chunk", type=int, default=512, help="prompt tokens per prefill call")
    ap.add_argument("--n-ctx", type=int, default=32768)
    ap.add_argument("--depth", type=int, default=4, help="drafts per round (k)")
    ap.add_argument("--profile-rounds", type=int, default=4)
    ap.add_argument("--cpu-baseline", type=int, default=1, help="0 skips the oracle timing")
    ap.add_argument("--cpu-rounds", type=int, default=5, help="timed whole oracle rounds of the CPU baseline")
    ap.add_argument("--cpu-configs", type=int, default=1, help="0 skips the oracle at configs 2-4's shapes")
    ap.add_argument("--gemm", type=int, default=1, help="0 skips the GEMM microbench (4 shapes x M)")
    ap.add_argument("--attn", type=int, default=1, help="0 skips the tree attention microbench")
    ap.add_argument("--legs", type=int, default=1,
                    help="0 skips the step-cost sweep, the oracle-drafts and the T = 0.7 legs")
    ap.add_argument("--run-tokens", type=int, default=512,
                    help="new tokens of the workload's greedy and T = 0.7 runs (the legs)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--sampler", type=int, default=1, help="0 skips the acceptance-sampler microbench")
    ap.add_argument("--sampler-only", action="store_true", help="run only the acceptance-sampler microbench")
    ap.add_argument("--gguf-load-only", type=int, default=0, metavar="LAYERS",
                    help="only time loading a seeded 27B-class GGUF file of LAYERS trunk layers")
    ap.add_argument("--replay", type=int, default=1, help="0: every round launches its kernels (no graph replay)")
    ap.add_argument("--calibrate-copy", type=int, default=0,
                    help="first copy 1 GiB on the device 3 times (a known-size kernel for HBM counters)")
    return ap.parse_args()


# ---------------------------------------------------------------- synthetic weights
def _fp16_bytes(torch, vals):
    return vals.to(torch.float16).view(torch.uint8).view(-1, 2)


def synth_quant(torch, qtype, n_rows, k, gen, device):
    """Random ggml blocks with plausible scales: weights roughly N(0, 0.02)-sized."""
    nb = n_rows * (k // 256)
    if qtype == Q4_K:
        raw = torch.randint(0, 256, (nb, 144), dtype=torch.uint8, device=device, generator=gen)
        u = torch.rand(nb, device=device, generator=gen)
        raw[:, 0:2] = _fp16_bytes(torch, 1.5e-4 + 1e-4 * u)          # d
        raw[:, 2:4] = _fp16_bytes(torch, 1.2e-3 + 6e-4 * u)          # dmin (keeps the mean near 0)
    elif qtype == Q8_0:
        nb = n_rows * (k // 32)
        raw = torch.randint(0, 256, (nb, 34), dtype=torch.uint8, device=device, generator=gen)
        u = torch.rand(nb, device=device, generator=gen)
        raw[:, 0:2] = _fp16_bytes(torch, 1.2e-4 + 6e-5 * u)          # d (codes are int8)
    else:
        raw = torch.randint(0, 256, (nb, 210), dtype=torch.uint8, device=device, generator=gen)
        u = torch.rand(nb, device=device, generator=gen)
        raw[:, 208:210] = _fp16_bytes(torch, 1.2e-5 + 6e-6 * u)      # d (scales are int8)
    return raw.view(-1)


def row_bytes(qtype, k):
    return k // 256 * 144 if qtype == Q4_K else k // 32 * 34 if qtype == Q8_0 else k // 256 * 210


def tensor_specs(hp):
    E, H, Hkv, hd, F, V = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["head_dim"], hp["n_ff"], hp["n_vocab"]
    specs = [("token_embd.weight", Q6_K, E, V), ("output.weight", Q6_K, E, V), ("output_norm.weight", F32, E, 1)]
    for il in range(hp["n_layer"] + (1 if hp["has_mtp"] else 0)):
        b = f"blk.{il}."
        specs += [(b + "attn_norm.weight", F32, E, 1), (b + "post_attention_norm.weight", F32, E, 1),
                  (b + "attn_q_norm.weight", F32, hd, 1), (b + "attn_k_norm.weight", F32, hd, 1),
                  (b + "attn_q.weight", Q4_K, E, 2 * H * hd), (b + "attn_k.weight", Q4_K, E, Hkv * hd),
                  (b + "attn_v.weight", Q4_K, E, Hkv * hd), (b + "attn_output.weight", Q4_K, H * hd, E),
                  (b + "ffn_gate.weight", Q4_K, E, F), (b + "ffn_up.weight", Q4_K, E, F),
                  (b + "ffn_down.weight", Q4_K, F, E)]
    if hp["has_mtp"]:
        b = f"blk.{hp['n_layer']}.nextn."
        specs += [(b + "eh_proj.weight", Q4_K, 2 * E, E), (b + "enorm.weight", F32, E, 1),
                  (b + "hnorm.weight", F32, E, 1)]
    return specs


def round_bytes(hp, n_kv, n_kv_mtp, depth, t):
    """Algorithmic bytes of one round: every weight the round streams once,
    the K and V rows it attends to as f16, and t rows of f32 activations in
    and out of each GEMM (small): (verify only, verify + depth MTP links)."""
    E, H, Hkv, hd, F = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["head_dim"], hp["n_ff"]
    layer = sum(row_bytes(q, k) * n for q, k, n in ((Q4_K, E, 2 * H * hd + 2 * Hkv * hd), (Q4_K, H * hd, E),
                                                    (Q4_K, E, 2 * F), (Q4_K, F, E)))
    acts = 4 * t * (E + (2 * H * hd + 2 * Hkv * hd) + H * hd + E + E + 2 * F + F + E)
    head = row_bytes(Q6_K, E) * hp["n_vocab"] + 4 * t * hp["n_vocab"]
    kv = lambda n: 2 * 2 * n * Hkv * hd
    verify = hp["n_layer"] * (layer + acts + kv(n_kv)) + head
    link = layer + acts + kv(n_kv_mtp) + row_bytes(Q4_K, 2 * E) * E + head
    return verify, verify + depth * link


def build_model(torch, ctx, hp, seed):
    from codpiece_amd.model import Model, make_hparams
    m = Model(ctx, make_hparams(**hp))
    gen = torch.Generator(device=ctx.torch_device)
    gen.manual_seed(seed)
    nbytes = 0
    for name, t, ne0, ne1 in tensor_specs(hp):
        if t == F32:
            data = torch.ones(ne0, dtype=torch.float32, device=ctx.torch_device)
        else:
            data = synth_quant(torch, t, ne1, ne0, gen, ctx.torch_device)
            nbytes += data.numel()
        m.set_tensor(name, t, data, ne0, ne1)
        del data
    m.ready()
    return m, nbytes


# ---------------------------------------------------------------- the fused loop
class Loop:
    """The fused loop's state (main.rs:803-913): last committed token and drafts."""

    def __init__(self, session, depth):
        self.s, self.depth = session, depth
        self.committed = 0
        self.accepted = self.proposed = self.rounds = 0

    def start(self, prompt, tail=64, bulk=64):
        split = max(0, len(prompt) - tail)
        for c in range(0, split, bulk):
            self.s.prefill(prompt[c:min(split, c + bulk)])
        out = self.s.step_fused_cached(prompt[split:], self.depth)
        n_past, mtp_past = self.s.pos
        self.s.set_pos(n_past, mtp_past + len(out.preds))
        last = len(out.preds) - 1
        self.last = out.preds[last]
        self.drafts = [out.chain[l][last] for l in range(self.depth)]

    def round(self):
        batch = [self.last] + self.drafts
        out = self.s.step_fused_cached(batch, self.depth)
        keep = 0
        while keep < len(self.drafts) and out.preds[keep] == self.drafts[keep]:
            keep += 1
        self.rounds += 1
        self.proposed += len(self.drafts)
        self.accepted += keep
        self.committed += keep + 1
        self.last = out.preds[keep]
        self.drafts = [out.chain[l][keep] for l in range(self.depth)]
        over = len(batch) - (keep + 1)
        n_past, mtp_past = self.s.pos
        self.s.set_pos(n_past - over, mtp_past + keep + 1)


# ---------------------------------------------------------------- CPU baseline
def physical_cores():
    """Physical cores of the host (distinct core/socket pairs in lscpu -p), or None."""
    import subprocess
    try:
        out = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    cores = {line.strip() for line in out.splitlines() if line.strip() and not line.startswith("#")}
    return len(cores) or None


def cpu_threads():
    """Host threads the CPU legs use: the process's CPU share (OMP_NUM_THREADS
    when the launcher sets one, else the affinity mask)."""
    aff = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(aff, int(env))) if env.isdigit() and int(env) > 0 else aff


def _host_pool(rng, pools, qtype, nbytes):
    """Random block bytes with fixed plausible scales, shared by every tensor
    of a type (each tensor's copy in the oracle model is its own memory)."""
    if qtype not in pools or pools[qtype].size < nbytes:
        raw = rng.integers(0, 2 ** 63, size=(nbytes + 7) // 8, dtype=np.uint64).view(np.uint8)[:nbytes].copy()
        if qtype == Q4_K:
            blk = raw.reshape(-1, 144)
            blk[:, 0:2] = np.frombuffer(np.float16(2e-4).tobytes(), np.uint8)
            blk[:, 2:4] = np.frombuffer(np.float16(1.5e-3).tobytes(), np.uint8)
        elif qtype == Q8_0:
            blk = raw.reshape(-1, 34)
            blk[:, 0:2] = np.frombuffer(np.float16(1.5e-4).tobytes(), np.uint8)
        else:
            blk = raw.reshape(-1, 210)
            blk[:, 208:210] = np.frombuffer(np.float16(1.5e-5).tobytes(), np.uint8)
        pools[qtype] = raw
    return pools[qtype][:nbytes]


def cpu_baseline(hp, threads, tokens_per_round, depth, seed, reps=5):
    """Whole verify rounds of the oracle (the C restatement of the reference's
    CPU ggml semantics under oracle/, not ggml itself) on the host: the
    27B-class model with synthetic weights in host memory, the session at
    n_past 4096 over a zero-filled KV cache (attention's cost does not depend
    on the values), rounds of [last] + `depth` drafts with the MTP chain,
    rewound after each; the median of `reps` rounds after one untimed."""
    from oracle import cpvo
    rng = np.random.default_rng(seed)
    t0 = time.perf_counter()
    m = cpvo.Model(hp)
    pools = {}
    for name, t, ne0, ne1 in tensor_specs(hp):
        if t == F32:
            m.set_tensor(name, t, np.ones(ne0, np.float32), ne0, ne1)
        else:
            m.set_tensor(name, t, _host_pool(rng, pools, t, ne1 * row_bytes(t, ne0)), ne0, ne1)
    pools.clear()
    build_s = time.perf_counter() - t0
    cpvo.set_threads(threads)
    n_past, mtp_past = 4096, 64
    s = cpvo.Session(m, n_past + 64)
    toks = rng.integers(0, hp["n_vocab"], size=depth + 1).tolist()
    times = []
    for r in range(reps + 1):
        s.set_pos(n_past, mtp_past)
        t1 = time.perf_counter()
        s.step_fused_cached(toks, depth)
        if r:
            times.append(time.perf_counter() - t1)
        print(f"[bench] cpu round {r}: {time.perf_counter() - t1:.2f} s", file=sys.stderr, flush=True)
    s.free()
    m.free()
    times.sort()
    round_s = times[len(times) // 2]
    return {
        "value": round(tokens_per_round / round_s, 4), "unit": "tok/s", "cores": threads, "kind": "port",
        "physical_cores_lscpu": physical_cores(), "round_s_median": round(round_s, 3),
        "round_s_all": [round(x, 3) for x in times],
        "sample": (f"the oracle (the repo's C restatement of the reference's CPU ggml path: exact-window GEMMs, "
                   f"exact-contract attention; not ggml, which is not vendored) timing {reps} whole verify rounds "
                   f"(median, one untimed first) of the same 27B-class model ({hp['n_layer']} layers, synthetic "
                   f"weights in host memory, built in {build_s:.0f} s) at n_past {n_past} over a zero-filled KV "
                   f"cache, {depth + 1} tokens + a {depth}-link MTP chain per round, on {threads} threads, at "
                   f"the GPU run's {tokens_per_round:.3f} committed tokens per round"),
    }


def cpu_configs(threads, seed):
    """The oracle's functions at configs 2-4's shapes on the host: the
    acceptance decision at B = 1 (T = 0.7, top-p 0.95, draft distribution),
    the Q4_K and Q8_0 GEMMs at M = 5 and the 16-node tree attention at
    context 8192; median of 3 timed calls each."""
    from oracle import cpvo
    rng = np.random.default_rng(seed + 5)
    pools = {}

    def med(fn, n=3):
        fn()
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[n // 2]

    out = {"threads": threads, "gemm_m5": {}}
    for qt, name in ((Q4_K, "q4_k"), (Q8_0, "q8_0")):
        for k, n in GEMM_SHAPES:
            wb = _host_pool(rng, pools, qt, n * row_bytes(qt, k))
            x = rng.normal(size=(5, k)).astype(np.float32)
            sec = med(lambda: cpvo.qgemm(qt, wb, x, threads))
            out["gemm_m5"][f"{name}_{k}x{n}"] = {"us": round(sec * 1e6, 1),
                                                 "GB_s": round(n * row_bytes(qt, k) / sec / 1e9, 2)}
    pools.clear()
    H, Hkv, hd, n_past = 40, 8, 128, 8192
    kc = cpvo.f32_to_f16_bits(rng.normal(size=(n_past + 16, Hkv * hd)).astype(np.float32))
    q = rng.normal(size=(16, H, hd)).astype(np.float32)
    sec = med(lambda: cpvo.attn(q, kc, kc, n_past, TREE16, np.float32(1 / np.sqrt(hd))))
    out["attention_tree16_ctx8192"] = {"us": round(sec * 1e6, 1),
                                       "GB_s": round(2 * kc.nbytes / sec / 1e9, 2)}
    V, k = 151936, 4
    pl = (rng.normal(size=(1, k + 1, V)) * 3).astype(np.float32)
    ql = (pl[:, :k] + rng.normal(size=(1, k, V))).astype(np.float32)
    dr = rng.integers(0, V, size=(1, k)).astype(np.int32)
    prm = cpvo.SamplerParams(temp=0.7, top_p=0.95)
    sec = med(lambda: cpvo.spec_accept(pl, dr, prm, cpvo.ACCEPT_REJECT, u=cpvo.philox_uniforms(seed, 1, k),
                                       q_logits=ql))
    out["acceptance_reject_draft_dist_b1"] = {"us": round(sec * 1e6, 1), "threads": 1}
    return out


# ---------------------------------------------------------------- sampler
def sampler_bench(torch, ctx, seed, reps=20):
    """The acceptance sampler at its headline shapes: target logits f32
    [B][k+1 = 5][151936] ~ N(0, 3) plus a +8 spike at a random id per row,
    draft logits = target + N(0, 1) over the k = 4 draft rows, drafts drawn
    from the draft distribution (T = 0.7, top-p 0.95); per call, rejection
    sampling with the draft distribution (the general rule), with one-hot
    drafts (the reference rule) and greedy argmax match, on Philox uniforms.
    Algorithmic bytes per call: the logit rows read once (target, plus the
    draft rows where used)."""
    from codpiece_amd.runtime import SamplerParams
    V, k = 151936, 4
    g = torch.Generator(device=ctx.torch_device).manual_seed(seed + 7)
    p = SamplerParams(temp=0.7, top_p=0.95)
    out = {}
    for B in (1, 4, 16):
        pl = torch.randn(B, k + 1, V, device=ctx.torch_device, generator=g) * 3.0
        spike = torch.randint(0, V, (B, k + 1), device=ctx.torch_device, generator=g)
        pl.scatter_add_(2, spike.unsqueeze(2), torch.full((B, k + 1, 1), 8.0, device=ctx.torch_device))
        ql = (pl[:, :k] + torch.randn(B, k, V, device=ctx.torch_device, generator=g)).contiguous()
        ids, probs, n = ctx.distribution(ql.view(B * k, V), p)
        u = torch.rand(B * k, device=ctx.torch_device, generator=g)
        cum = torch.cumsum(probs, dim=1)
        pick = torch.searchsorted(cum, (u * cum.gather(1, (n - 1).long().unsqueeze(1)).squeeze(1)).unsqueeze(1))
        pick = torch.minimum(pick.squeeze(1), (n - 1).long())
        drafts = ids.gather(1, pick.unsqueeze(1)).view(B, k).to(torch.int32)
        res = {}
        for name, mode, q, bytes_ in (("reject_draft_dist", 1, ql, 4.0 * V * (B * (k + 1) + B * k)),
                                      ("reject_one_hot", 1, None, 4.0 * V * B * (k + 1)),
                                      ("greedy", 0, None, 4.0 * V * B * (k + 1))):
            prm = p if mode else SamplerParams()
            for _ in range(3):
                ctx.spec_accept(pl, drafts, prm, mode, q_logits=q, philox_seed=seed)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(reps):
                ctx.spec_accept(pl, drafts, prm, mode, q_logits=q, philox_seed=seed + i)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / reps * 1e3
            res[name] = {"us_per_call": round(us, 1), "GB_s": round(bytes_ / (us * 1e-6) / 1e9, 1),
                         "MB_per_call": round(bytes_ / 1e6, 2)}
        out[f"B={B}"] = res
        print(f"[bench] sampler B={B}: " + ", ".join(f"{k2} {v['us_per_call']} us" for k2, v in res.items()),
              file=sys.stderr, flush=True)
    return out


def gemm_bench(torch, ctx, seed, rotate_bytes=512e6):
    """The verify GEMM at its shapes: Q4_K and Q8_0 weights (random blocks
    with plausible scales; Q6_K too, the head's and a Q4_K_M file's other
    type) x f32 activations ~N(0, 1) of M rows, for each of
    GEMM_SHAPES and M in {1, 5, 8, 16}, and at 256 rows (a prefill chunk's:
    `TOP_s` is its int8 rate); `kernel` "wide" marks the launches the library
    gave its wide kernels (Q6_K and Q8_0 from 9 rows, Q4_K from 17).  Each shape's weights are uploaded in
    enough copies to cover `rotate_bytes` (more than the 256 MB last-level
    cache), and consecutive calls rotate through them, so every call streams
    its weights from HBM.  `us` is the GEMM kernels' time per call (the
    recorded launches replayed back to back between one event pair, as for
    the roofline); `us_call` adds the activation quantization and the
    finalize kernel (whole calls back to back, one event pair).  Algorithmic
    bytes per call: the weight blocks, the quantized activations and the f32
    outputs."""
    gen = torch.Generator(device=ctx.torch_device).manual_seed(seed + 11)
    dev = ctx.torch_device
    out = {}
    for qt, name in ((Q4_K, "q4_k"), (Q8_0, "q8_0"), (Q6_K, "q6_k")):
        cls = "qgemm_" + name
        for k, n in GEMM_SHAPES:
            wbytes = n * row_bytes(qt, k)
            copies = max(2, int(np.ceil(rotate_bytes / wbytes)))
            ws = []
            for _ in range(copies):
                raw = synth_quant(torch, qt, n, k, gen, dev)
                ws.append(ctx.upload_weight(qt, raw, n, k))
                del raw
            res = {"weights_MB": round(wbytes / 1e6, 2), "copies_rotated": copies}
            for M in (1, 5, 8, 16, 256):
                x = torch.randn(M, k, device=dev, generator=gen)
                y = torch.empty(M, n, device=dev)
                for w in ws[:2]:
                    ctx.qgemm(w, x, y)
                ctx.profile_start()
                for w in ws:
                    ctx.qgemm(w, x, y)
                prof = ctx.profile_stop()
                # (the skinny or the wide kernel's class, as the library chose by rows)
                mcls = cls if prof[cls][0] > 0 else cls + "_wide"
                launches = prof[mcls][0]
                ms, b = ctx.profile_replay(mcls, reps=3)
                per = launches / copies
                us = ms * 1e3 * per
                gbs = b * per / (us * 1e-6) / 1e9
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for w in ws:
                    ctx.qgemm(w, x, y)
                e1.record()
                torch.cuda.synchronize()
                res[f"M={M}"] = {"us": round(us, 2), "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                                 "MB": round(b * per / 1e6, 2), "launches": per,
                                 "us_call": round(e0.elapsed_time(e1) * 1e3 / copies, 2)}
                if mcls != cls:
                    res[f"M={M}"]["kernel"] = "wide"
                if M >= 32:
                    res[f"M={M}"]["TOP_s"] = round(2.0 * M * n * k / (us * 1e-6) / 1e12, 1)
            out[f"{name} {k}x{n}"] = res
            print(f"[bench] gemm {name} {k}x{n}: " + ", ".join(f"{m} {v['us']} us ({v['frac']:.2f})"
                                                              for m, v in res.items() if m.startswith("M=")),
                  file=sys.stderr, flush=True)
            for w in ws:
                w.free()
    return out


def attn_bench(torch, ctx, seed, reps=10):
    """Tree-verify attention: 40 Q / 8 KV heads x 128 over an f16 KV cache
    ~N(0, 1) of n_ctx rows plus the 16 nodes of TREE16 (ancestor-only mask),
    at n_ctx 8192 and 32768; each call replayed `reps` times between one
    event pair.  Algorithmic bytes: K and V rows once, q in and the output."""
    gen = torch.Generator(device=ctx.torch_device).manual_seed(seed + 13)
    dev = ctx.torch_device
    H, Hkv, hd, t = 40, 8, 128, len(TREE16)
    par = torch.tensor(TREE16, dtype=torch.int32, device=dev)
    out = {}
    for n_ctx in (8192, 32768):
        rows = n_ctx + t
        kc = torch.randn(rows, Hkv * hd, device=dev, generator=gen).half().view(torch.int16)
        vt = torch.zeros(Hkv * hd, (rows + 7) // 8 * 8, dtype=torch.float16, device=dev)
        vt[:, :rows] = torch.randn(Hkv * hd, rows, device=dev, generator=gen).half()
        vt = vt.view(torch.int16)
        q = torch.randn(t, H, hd, device=dev, generator=gen)
        o = torch.empty(t, H * hd, device=dev)
        scale = 1.0 / float(np.sqrt(hd))
        ctx.attn(q, kc, vt, n_ctx, par, Hkv, scale, out=o)
        ctx.profile_start()
        ctx.attn(q, kc, vt, n_ctx, par, Hkv, scale, out=o)
        ctx.profile_stop()
        ms, b = ctx.profile_replay("attention", reps=reps)
        gbs = b / (ms * 1e-3) / 1e9
        out[f"ctx={n_ctx}"] = {"us": round(ms * 1e3, 2), "MB": round(b / 1e6, 2), "GB_s": round(gbs, 1),
                               "frac": round(gbs / HBM_PEAK_GBS, 4)}
        print(f"[bench] attention tree16 ctx {n_ctx}: {ms * 1e3:.1f} us ({gbs:.0f} GB/s)", file=sys.stderr,
              flush=True)
        del kc, vt
    return out


def step_cost_sweep(torch, sess, stream, toks, reps=5):
    """The verify step's device time against the tokens it carries
    (crates/codpiece-cli/src/main.rs:549-629, stepcost): verify-only rounds
    (no MTP chain) of T tokens in a chain, median of `reps`, rewound after
    each."""
    n_past, mtp_past = sess.pos
    out = {}
    for T in (1, 2, 4, 8, 16):
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            sess.step_fused_cached(toks[:T], 0)
            b.record(stream)
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
            sess.set_pos(n_past, mtp_past)
        ts.sort()
        out[f"T={T}"] = round(ts[len(ts) // 2] * 1e3, 1)
    print("[bench] step cost (us): " + ", ".join(f"{k} {v}" for k, v in out.items()), file=sys.stderr, flush=True)
    return out


def oracle_drafts_leg(sess, prompt, depth, chunk, n_gen=64):
    """Accepted tokens/s when every draft is right: the plain greedy stream
    (depth 0) is generated first, then the fused loop runs with drafts taken
    from that stream (an oracle drafter), so each round accepts all `depth`
    drafts and commits depth + 1 tokens.  The committed stream must equal the
    plain one (losslessness)."""
    from codpiece_amd.model import fused_generate
    sess.set_pos(0, 0)
    plain, _ = fused_generate(sess, prompt, n_gen, 0, tail=64, bulk=chunk)

    def drafter(committed, chain):
        n = len(committed)
        return plain[n:n + depth]

    sess.set_pos(0, 0)
    toks, st = fused_generate(sess, prompt, n_gen, depth, tail=64, bulk=chunk, drafter=drafter)
    return {"tokens": len(toks), "rounds": st.rounds, "acceptance": round(st.accepted / max(1, st.proposed), 4),
            "tokens_per_round": round((len(toks) - 1) / max(1, st.rounds), 3),
            "decode_s": round(st.decode_s, 4), "tok_s": round((len(toks) - 1) / st.decode_s, 2),
            "stream_equals_plain_greedy": toks == plain}


def greedy_leg(sess, prompt, depth, chunk, n_gen=512):
    """The workload's greedy run at its full length: the fused loop
    (main.rs:843-929) from a fresh prefill of the prompt, n_gen tokens."""
    from codpiece_amd.model import fused_generate
    sess.set_pos(0, 0)
    toks, st = fused_generate(sess, prompt, n_gen, depth, tail=64, bulk=chunk)
    return {"tokens": len(toks), "rounds": st.rounds, "acceptance": round(st.accepted / max(1, st.proposed), 4),
            "tokens_per_round": round((len(toks) - 1) / max(1, st.rounds), 3), "prefill_s": round(st.prefill_s, 3),
            "decode_s": round(st.decode_s, 4), "tok_s": round((len(toks) - 1) / st.decode_s, 2)}


def sampled_leg(sess, prompt, depth, chunk, seed, n_gen=512):
    """The workload's T = 0.7 / top-p 0.95 run at its full length: the engine's
    sampled speculative loop (rejection rule on the device with Philox
    uniforms, MTP chain drafts, the post-commit re-draft at the engine's
    defaults: 3 links, softmax-peak gate 0.75), n_gen tokens."""
    from codpiece_amd import _lib
    from codpiece_amd.model import sampled_generate
    from codpiece_amd.runtime import SamplerParams
    sess.set_pos(0, 0)
    toks, st = sampled_generate(sess, prompt, n_gen, depth, SamplerParams(temp=0.7, top_p=0.95),
                                _lib.ACCEPT_REJECT, seed=seed, tail=64, bulk=chunk)
    return {"tokens": len(toks), "rounds": st.rounds, "acceptance": round(st.accepted / max(1, st.proposed), 4),
            "tokens_per_round": round((len(toks) - 1) / max(1, st.rounds), 3), "prefill_s": round(st.prefill_s, 3),
            "decode_s": round(st.decode_s, 4), "tok_s": round((len(toks) - 1) / st.decode_s, 2),
            "redraft_rounds": st.redraft_rounds, "redraft_links": st.redraft_links}


def prefill_gemm_stats(ctx, prof, hp, rows):
    """The wide Q4_K GEMM of one prefill chunk: launches, replayed time per
    launch, and int8 throughput against the dense MFMA peak (multiply-adds
    per token and layer: the q|gate|k|v, wo, gate|up and down projections)."""
    n, ms, _ = prof.get("qgemm_q4_k_wide", (0, 0.0, 0.0))
    if not n:
        return None
    rep_ms, rep_bytes = ctx.profile_replay("qgemm_q4_k_wide", reps=3)
    E, F = hp["n_embd"], hp["n_ff"]
    attn = 2 * hp["n_head"] * hp["head_dim"] + 2 * hp["n_head_kv"] * hp["head_dim"]
    macs = rows * hp["n_layer"] * E * (attn + E + 2 * F + F)
    tops = 2.0 * macs / (n * rep_ms * 1e-3) / 1e12
    return {"rows": rows, "launches": n, "us_per_launch_replayed": round(rep_ms * 1e3, 2),
            "us_per_launch_event_bracketed": round(ms / n * 1e3, 2),
            "int8_TOP_s": round(tops, 1), "roofline": {"bound": "mfma", "peak": INT8_MFMA_PEAK_TOPS,
                                                       "unit": "TOP/s", "frac": round(tops / INT8_MFMA_PEAK_TOPS, 4)}}


# ---------------------------------------------------------------- main
def gguf_load_bench(ctx, layers, seed):
    """Weights::load of a seeded 27B-class qwen35 file (Q4_K linears, Q6_K
    embedding and head, `layers` trunk layers and the MTP layer): the file is
    written to a temporary directory, then loaded (file read, host-to-device
    copy and repack of every tensor) and timed end to end."""
    import tempfile
    from codpiece_amd import gguf
    from codpiece_amd.model import Model
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.gguf")
        t0 = time.perf_counter()
        gguf.write_seeded_model(path, layers, HP["n_embd"], HP["n_head"], HP["n_head_kv"], HP["head_dim"],
                                HP["n_ff"], HP["n_vocab"], n_rot=HP["n_rot"], rope_sections=HP["rope_sections"],
                                seed=seed, qtype=gguf.Q4_K, head_type=gguf.Q6_K)
        size = os.path.getsize(path)
        print(f"[bench] wrote {size / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
        ctx.sync()
        t0 = time.perf_counter()
        m = Model.from_gguf(ctx, path)
        ctx.sync()
        s = time.perf_counter() - t0
        m.free()
    return {"layers": layers, "file_GB": round(size / 1e9, 3), "seconds": round(s, 3), "GB_s": round(size / 1e9 / s, 2)}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: the verify step runs on a single GPU (the 27B-class "
              f"model is resident in one GPU's HBM); --gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from codpiece_amd.model import Session
    from codpiece_amd.runtime import Context

    hp = dict(HP, n_layer=args.layers)
    torch.cuda.set_device(0)
    ctx = Context(0)
    if args.sampler_only:
        print(json.dumps({"sampler": sampler_bench(torch, ctx, args.seed)}), flush=True)
        ctx.close()
        return 0
    if args.gguf_load_only:
        print(json.dumps({"gguf_load": gguf_load_bench(ctx, args.gguf_load_only, args.seed)}), flush=True)
        ctx.close()
        return 0
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=ctx.torch_device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    t0 = time.perf_counter()
    model, wbytes = build_model(torch, ctx, hp, args.seed)
    torch.cuda.synchronize()
    print(f"[bench] model built: {wbytes / 1e9:.2f} GB quantized weights in {time.perf_counter() - t0:.1f} s",
          file=sys.stderr, flush=True)
    chunk = max(64, min(args.prefill_chunk, 4096))
    sess = Session(model, args.n_ctx, max_batch=chunk)
    sess.set_replay(bool(args.replay))
    g = torch.Generator().manual_seed(args.seed + 1)
    prompt = torch.randint(0, hp["n_vocab"], (args.prompt,), generator=g).tolist()
    # the prefill's GEMMs over one chunk, each launch timed, then rewound
    pchunk = min(chunk, args.prompt)
    sess.prefill(prompt[:pchunk])      # (sizes the workspaces the profiled launches keep using)
    sess.set_pos(0, 0)
    ctx.profile_start()
    sess.prefill(prompt[:pchunk])
    pprof = ctx.profile_stop()
    sess.set_pos(0, 0)
    prefill_gemm = prefill_gemm_stats(ctx, pprof, hp, pchunk)
    loop = Loop(sess, args.depth)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    loop.start(prompt, bulk=chunk)
    e1.record()
    torch.cuda.synchronize()
    prefill_wall = time.perf_counter() - t0
    prefill_dev = e0.elapsed_time(e1) * 1e-3
    print(f"[bench] prefill of {args.prompt} tokens in {chunk}-token chunks: {prefill_wall:.2f} s "
          f"({prefill_dev:.2f} s device, {args.prompt / prefill_dev:.0f} tok/s)", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        loop.round()
    # timed rounds: device time of each round by events on the library's stream
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    c0 = loop.committed
    acc0, prop0 = loop.accepted, loop.proposed
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        evs[i][0].record(stream)
        loop.round()
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    committed = loop.committed - c0
    dev_ms = sorted(a.elapsed_time(b) for a, b in evs)
    print(f"[bench] {args.steps} rounds in {wall:.3f} s, {committed} tokens", file=sys.stderr, flush=True)

    # verify-only rounds (depth 0), rewound afterwards
    n_past, mtp_past = sess.pos
    vo = []
    for _ in range(max(3, args.steps // 4)):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        sess.step_fused_cached([loop.last] + loop.drafts, 0)
        b.record(stream)
        torch.cuda.synchronize()
        vo.append(a.elapsed_time(b))
        sess.set_pos(n_past, mtp_past)
    vo.sort()
    # the round's algorithmic bytes over its device time (the verify rows attend
    # to n_past + t rows; the MTP links to their own cache, mtp_past + t)
    t_round = 1 + args.depth
    vb, rb = round_bytes(hp, n_past + t_round, mtp_past + t_round, args.depth, t_round)
    vo_s, round_s = vo[len(vo) // 2] * 1e-3, dev_ms[len(dev_ms) // 2] * 1e-3
    round_stats = {"verify_only_GB": round(vb / 1e9, 3), "verify_only_GB_s": round(vb / vo_s / 1e9, 1),
                   "verify_only_frac": round(vb / vo_s / 1e9 / HBM_PEAK_GBS, 4),
                   "round_GB": round(rb / 1e9, 3), "round_GB_s": round(rb / round_s / 1e9, 1),
                   "round_frac": round(rb / round_s / 1e9 / HBM_PEAK_GBS, 4)}
    print(f"[bench] round bytes: {round_stats}", file=sys.stderr, flush=True)

    # full rounds with the draft head over an 8192-token shortlist, rewound afterwards
    cands = np.arange(8192, dtype=np.int32)
    sl = []
    for _ in range(max(3, args.steps // 4)):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        sess.step_fused_cached([loop.last] + loop.drafts, args.depth, cands=cands)
        b.record(stream)
        torch.cuda.synchronize()
        sl.append(a.elapsed_time(b))
        sess.set_pos(n_past, mtp_past)
    sl.sort()

    # draft trees: the canonical 16-node tree (widths 4, 6, 3, 3) verified, then
    # its deepest leftmost path committed; rewound afterwards
    tree = [-1, -1, -1, -1, 0, 0, 0, 1, 1, 1, 4, 4, 4, 10, 10, 10]
    ttoks = torch.randint(0, hp["n_vocab"], (len(tree),), generator=g).tolist()
    tv, tc = [], []
    for _ in range(max(3, args.steps // 4)):
        a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        a.record(stream)
        sess.verify_tree(ttoks, tree)
        b.record(stream)
        sess.commit_branch([0, 4, 10, 13])
        c.record(stream)
        torch.cuda.synchronize()
        tv.append(a.elapsed_time(b))
        tc.append(b.elapsed_time(c))
        sess.set_pos(n_past, mtp_past)
    tv.sort()
    tc.sort()

    step_cost = None
    if args.legs:
        sweep_toks = [loop.last] + loop.drafts
        sweep_toks += torch.randint(0, hp["n_vocab"], (16 - len(sweep_toks),), generator=g).tolist()
        step_cost = step_cost_sweep(torch, sess, stream, sweep_toks)

    # per-class kernel timing over extra rounds (events between launches: not in the timed region)
    ctx.profile_start()
    for _ in range(args.profile_rounds):
        loop.round()
    prof = ctx.profile_stop()
    dom = max(prof, key=lambda k: prof[k][1])
    # the recorded launches of each class, replayed back to back between one event pair
    replay = {k: ctx.profile_replay(k, reps=3) for k, v in prof.items() if v[0]}
    rep_ms, rep_bytes = replay[dom]
    achieved = rep_bytes / (rep_ms * 1e-3) / 1e9

    # HBM bytes per launch by class, from rocprofv3 FETCH_SIZE / WRITE_SIZE
    # passes at this workload's shape (profiles/traffic_hbm_27b_q4k_ctx4096.md)
    traffic_table = {}
    tpath = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic_table = json.load(f)
    traffic = traffic_table.get(dom)

    oracle_drafts = sampled = greedy = None
    if args.legs:
        oracle_drafts = oracle_drafts_leg(sess, prompt, args.depth, chunk)
        print(f"[bench] oracle drafts: {oracle_drafts}", file=sys.stderr, flush=True)
        greedy = greedy_leg(sess, prompt, args.depth, chunk, args.run_tokens)
        print(f"[bench] greedy run: {greedy}", file=sys.stderr, flush=True)
        sampled = sampled_leg(sess, prompt, args.depth, chunk, args.seed, args.run_tokens)
        print(f"[bench] T=0.7 run: {sampled}", file=sys.stderr, flush=True)
    gemm = gemm_bench(torch, ctx, args.seed) if args.gemm else None
    attn = attn_bench(torch, ctx, args.seed) if args.attn else None
    sampler = sampler_bench(torch, ctx, args.seed) if args.sampler else None

    threads = cpu_threads()
    cpu = cpu_cfg = None
    if args.cpu_baseline:
        cpu = cpu_baseline(hp, threads, committed / args.steps, args.depth, args.seed, reps=args.cpu_rounds)
    if args.cpu_configs:
        cpu_cfg = cpu_configs(threads, args.seed)

    value = committed / wall
    line = {
        "metric": "verify-step µs + accepted tok/s, 27B-class Q4_K, draft k=4, 1 MI355X",
        "value": round(value, 3), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic (random-init weights and prompt)",
        "config": {"workload": (f"27B-class qwen35-layout random-init model: {hp['n_layer']} layers, d_model 5120, "
                                f"40/8 heads x 128, FFN 17408, vocab 151936, Q4_K linears, Q6_K embedding/output, "
                                f"1 MTP layer; {args.prompt}-token random prompt, context {args.n_ctx}; "
                                f"greedy speculative decode, k={args.depth}"),
                   "k": args.depth, "context": args.n_ctx, "prompt": args.prompt},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "detail": {
            "round_device_us_median": round(dev_ms[len(dev_ms) // 2] * 1e3, 1),
            "round_bytes": round_stats,
            "verify_only_device_us_median": round(vo[len(vo) // 2] * 1e3, 1),
            "round_shortlist_8192_device_us_median": round(sl[len(sl) // 2] * 1e3, 1),
            "tree_verify_16_device_us_median": round(tv[len(tv) // 2] * 1e3, 1),
            "tree_commit_4_device_us_median": round(tc[len(tc) // 2] * 1e3, 1),
            "acceptance": round((loop.accepted - acc0) / max(1, loop.proposed - prop0), 4),
            "tokens_per_round": round(committed / args.steps, 3),
            "replay": {"on": bool(args.replay), "captured": sess.replay_stats[0], "replayed": sess.replay_stats[1]},
            "kernel_classes": {k: {"launches_per_round": v[0] / args.profile_rounds,
                                   "GB_per_launch": round(v[2] / v[0] / 1e9, 5),
                                   "us_per_launch_replayed": round(replay[k][0] * 1e3, 2),
                                   "GB_s_replayed": round(replay[k][1] / (replay[k][0] * 1e-3) / 1e9, 1),
                                   "us_per_launch_event_bracketed": round(v[1] / v[0] * 1e3, 2),
                                   "hbm_bytes_per_launch": traffic_table.get(k)}
                               for k, v in prof.items() if v[0]},
            "profiled_rounds": args.profile_rounds,
            "prefill": {"tokens": args.prompt, "chunk": chunk, "wall_s": round(prefill_wall, 3),
                        "device_s": round(prefill_dev, 3), "tokens_per_s": round(args.prompt / prefill_dev, 1),
                        "gemm_q4_k_wide": prefill_gemm},
            "acceptance_sampler": sampler,
            "step_cost_us": step_cost,
            "oracle_drafts": oracle_drafts,
            "greedy_run": greedy,
            "sampled_T0.7_top_p0.95": sampled,
            "gemm": gemm,
            "attention_tree16": attn,
            "cpu_configs": cpu_cfg,
        },
    }
    print(json.dumps(line), flush=True)
    sess.free()
    model.free()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
