"""Host mirror of codpiece-model's verify-round interface over the C ABI.

`Model` loads tensors by GGUF name (Weights::load, crates/codpiece-model/src/
lib.rs:128-311); `Session` owns the KV caches and positions (Session::new_spec,
qwen35.rs:528-649); `Session.step_fused_cached` is Qwen35::step_fused_cached
(qwen35.rs:1693-1948) and returns a `FusedOut` (qwen35.rs:817-828);
`fused_generate` is the CLI's fused greedy speculative loop (crates/codpiece-
cli/src/main.rs:643-931); `sampled_generate` is the engine's sampled
speculative loop (crates/codpiece-server/src/engine.rs:1922-2039,
2212-2542).  All arithmetic runs in libcpv.so.
"""
import ctypes
from collections import deque
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from ._lib import CpvError, DraftOut, Hparams, RoundOut


def make_hparams(n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_rot=None,
                 rope_sections=(0, 0, 0, 0), rms_eps=1e-6, freq_base=1e6, has_mtp=True):
    hp = Hparams()
    hp.n_layer, hp.n_embd, hp.n_head, hp.n_head_kv = n_layer, n_embd, n_head, n_head_kv
    hp.head_dim, hp.n_ff, hp.n_vocab = head_dim, n_ff, n_vocab
    hp.n_rot = head_dim if n_rot is None else n_rot
    for i, v in enumerate(rope_sections):
        hp.rope_sections[i] = v
    hp.rms_eps, hp.freq_base, hp.has_mtp = rms_eps, freq_base, int(has_mtp)
    return hp


class Model:
    def __init__(self, ctx, hp):
        self.ctx, self.hp = ctx, hp
        h = ctypes.c_void_p()
        ctx._check(ctx.lib.cpv_model_create(ctx.h, ctypes.byref(hp), ctypes.byref(h)))
        self.h = h

    @classmethod
    def from_gguf(cls, ctx, path):
        """Weights::load of a qwen35 GGUF file (all-attention layout)."""
        self = cls.__new__(cls)
        h = ctypes.c_void_p()
        ctx._check(ctx.lib.cpv_model_load_gguf(ctx.h, str(path).encode(), ctypes.byref(h)))
        self.ctx, self.h = ctx, h
        from .gguf import hparams
        self.hp = hparams(path)
        return self

    def set_tensor(self, name, qtype, data, ne0, ne1):
        """data: numpy (host bytes) or a cuda tensor (device bytes), ggml ne order."""
        if isinstance(data, torch.Tensor):
            ptr, dev = ctypes.c_void_p(data.data_ptr()), 1
        else:
            data = np.ascontiguousarray(data)
            ptr, dev = data.ctypes.data_as(ctypes.c_void_p), 0
        self.ctx._check(self.ctx.lib.cpv_model_set_tensor(self.h, name.encode(), qtype, ptr, dev, ne0, ne1))

    def ready(self):
        self.ctx._check(self.ctx.lib.cpv_model_ready(self.h))

    def free(self):
        if self.h:
            self.ctx.lib.cpv_model_free(self.h)
            self.h = None


@dataclass
class FusedOut:
    preds: list
    chain: list = field(default_factory=list)   # [depth][t]
    conf: list = field(default_factory=list)    # [depth][t]
    logits: object = None                       # torch [t][V] on the device, when wanted
    hidden: object = None                       # torch [t][E] on the device, when wanted


@dataclass
class DraftResult:
    """One standalone draft link: the draft (argmax), the gate's verdict, the
    link's hidden row as a device pointer for the next link (session memory,
    valid until the session's next call), and, when asked, copies of the
    logits and hidden."""
    draft: int
    keep: bool
    hidden_ptr: int
    logits: object = None
    hidden: object = None


class Session:
    def __init__(self, model, n_ctx, max_batch=64):
        self.model, self.ctx = model, model.ctx
        h = ctypes.c_void_p()
        self.ctx._check(self.ctx.lib.cpv_session_create(model.h, n_ctx, max_batch, ctypes.byref(h)))
        self.h = h
        self.max_batch = max_batch
        self._tok = torch.empty(max_batch, dtype=torch.int32, device=self.ctx.torch_device)
        # pinned host staging: the tokens go up and a round's ids and
        # confidences come down asynchronously, with one wait per round
        self._tok_h = torch.empty(max_batch, dtype=torch.int32, pin_memory=True)
        self._ids_h = torch.empty(0, dtype=torch.int32, pin_memory=True)
        self._conf_h = torch.empty(0, dtype=torch.float32, pin_memory=True)
        self._tok_ev = None

    @property
    def pos(self):
        a, b = ctypes.c_int64(), ctypes.c_int64()
        self.ctx._check(self.ctx.lib.cpv_session_get_pos(self.h, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def set_pos(self, n_past, mtp_past):
        self.ctx._check(self.ctx.lib.cpv_session_set_pos(self.h, n_past, mtp_past))

    def set_attn_tap(self, tap):
        """Copy every attention output of the next calls into `tap` (a float32
        cuda tensor), blocks in call order; None clears it."""
        if tap is None:
            self.ctx._check(self.ctx.lib.cpv_session_set_attn_tap(self.h, None, 0))
        else:
            self._tap = tap
            self.ctx._check(self.ctx.lib.cpv_session_set_attn_tap(self.h, ctypes.c_void_p(tap.data_ptr()),
                                                                  tap.numel()))

    def set_replay(self, on):
        """Replay greedy rounds from per-shape HIP graphs (on by default)."""
        self.ctx._check(self.ctx.lib.cpv_session_set_replay(self.h, 1 if on else 0))

    @property
    def replay_stats(self):
        """(rounds captured as graphs, rounds replayed) since the session was made."""
        c, r = ctypes.c_int64(), ctypes.c_int64()
        self.ctx._check(self.ctx.lib.cpv_session_replay_stats(self.h, ctypes.byref(c), ctypes.byref(r)))
        return c.value, r.value

    @property
    def n_past(self):
        return self.pos[0]

    @property
    def mtp_past(self):
        return self.pos[1]

    def _tokens(self, tokens):
        # the staging buffer is rewritten once the previous call's copy out of
        # it has run (calls that do not wait for their results, such as
        # prefill chunks, may still have it queued)
        t = len(tokens)
        if self._tok_ev is not None:
            self._tok_ev.synchronize()
        self._tok_h[:t].numpy()[:] = np.asarray(tokens, dtype=np.int32)
        with torch.cuda.stream(self.ctx.stream):
            self._tok[:t].copy_(self._tok_h[:t], non_blocking=True)
            self._tok_ev = torch.cuda.Event()
            self._tok_ev.record(self.ctx.stream)
        return t

    def _fetch_round(self, out, t, depth):
        """The round's preds [t], chain [depth][t] and confidences [depth][t]
        copied down on the stream, then one wait."""
        n_ids = (1 + depth) * t
        if self._ids_h.numel() < n_ids:
            self._ids_h = torch.empty(n_ids, dtype=torch.int32, pin_memory=True)
        if self._conf_h.numel() < max(depth * t, 1):
            self._conf_h = torch.empty(max(depth * t, 1), dtype=torch.float32, pin_memory=True)
        dev = self.ctx.torch_device
        with torch.cuda.stream(self.ctx.stream):
            self._ids_h[:t].copy_(_device_view(out.preds_dev, t, torch.int32, dev), non_blocking=True)
            if depth:
                self._ids_h[t:n_ids].copy_(_device_view(out.chain_dev, depth * t, torch.int32, dev),
                                           non_blocking=True)
                self._conf_h[:depth * t].copy_(_device_view(out.conf_dev, depth * t, torch.float32, dev),
                                               non_blocking=True)
        self.ctx.stream.synchronize()
        ids = self._ids_h[:n_ids].tolist()
        preds = ids[:t]
        chain = [ids[t + l * t:t + (l + 1) * t] for l in range(depth)]
        conf = self._conf_h[:depth * t].view(depth, t).tolist() if depth else []
        return preds, chain, conf

    def prefill(self, tokens):
        t = self._tokens(tokens)
        self.ctx._check(self.ctx.lib.cpv_prefill(self.h, ctypes.c_void_p(self._tok.data_ptr()), t))

    def mtp_draft(self, hidden, token, pos, p_min=0.0, want=False):
        """Qwen35::mtp_draft (qwen35.rs:2086-2192): one draft link from the
        hidden row `hidden` (a cuda tensor of n_embd floats, or the device
        pointer of a previous link's hidden_ptr) and `token` at rope position
        `pos`; mtp_past advances by 1.  The gate is the re-draft's softmax-peak
        test at p_min (engine.rs:2598-2606; 0 = no gate)."""
        if isinstance(hidden, torch.Tensor):
            assert hidden.is_cuda and hidden.dtype == torch.float32 and hidden.numel() == self.model.hp.n_embd
            hidden = hidden.contiguous()
            hp = hidden.data_ptr()
        else:
            hp = int(hidden)
        out = DraftOut()
        self.ctx._check(self.ctx.lib.cpv_mtp_draft(self.h, ctypes.c_void_p(hp), int(token), int(pos), float(p_min),
                                                   ctypes.byref(out)))
        if self._ids_h.numel() < 2:
            self._ids_h = torch.empty(16, dtype=torch.int32, pin_memory=True)
        dev = self.ctx.torch_device
        with torch.cuda.stream(self.ctx.stream):
            self._ids_h[:1].copy_(_device_view(out.draft_dev, 1, torch.int32, dev), non_blocking=True)
            self._ids_h[1:2].copy_(_device_view(out.keep_dev, 1, torch.int32, dev), non_blocking=True)
        self.ctx.stream.synchronize()
        d, k = self._ids_h[:2].tolist()
        logits = hid = None
        if want:
            V, E = self.model.hp.n_vocab, self.model.hp.n_embd
            logits = _device_view(out.logits_dev, V, torch.float32, dev).clone()
            hid = _device_view(out.hidden_dev, E, torch.float32, dev).clone()
        return DraftResult(int(d), bool(k), int(out.hidden_dev), logits, hid)

    def step_fused_cached(self, tokens, depth, want_logits=False, noise=None, cands=None):
        """Verify `tokens` and chain `depth` drafts; greedy in-graph argmax,
        gumbel argmax when `noise` ([t][V] device tensor) is given; the draft
        head over the shortlist `cands` (token ids) when given."""
        t = self._tokens(tokens)
        out = RoundOut()
        if noise is not None:
            noise = _as_device(noise, self.ctx.torch_device)
        nz = None if noise is None else ctypes.c_void_p(noise.data_ptr())
        if cands is None:
            self.ctx._check(self.ctx.lib.cpv_verify_step(self.h, ctypes.c_void_p(self._tok.data_ptr()), t, depth,
                                                         nz, ctypes.byref(out)))
        else:
            c = np.ascontiguousarray(cands, dtype=np.int32)
            self.ctx._check(self.ctx.lib.cpv_verify_step_cands(
                self.h, ctypes.c_void_p(self._tok.data_ptr()), t, depth, nz,
                c.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), int(c.size), ctypes.byref(out)))
        V, E = self.model.hp.n_vocab, self.model.hp.n_embd
        preds, chain, conf = self._fetch_round(out, t, depth)
        logits = hidden = None
        if want_logits:
            logits = _device_view(out.logits_dev, t * V, torch.float32, self.ctx.torch_device).view(t, V).clone()
            hidden = _device_view(out.hidden_dev, t * E, torch.float32, self.ctx.torch_device).view(t, E).clone()
        return FusedOut(preds, chain, conf, logits, hidden)

    def verify_tree(self, tokens, parent, want_logits=False, noise=None):
        """Verify a draft tree: tokens[i] with parent[i] (-1: a child of the
        context; parents precede children).  Returns the argmax of each node's
        logits (and the logits and hidden rows when asked)."""
        t = self._tokens(tokens)
        par = (ctypes.c_int32 * t)(*[int(p) for p in parent])
        out = RoundOut()
        nz = None if noise is None else ctypes.c_void_p(noise.data_ptr())
        self.ctx._check(self.ctx.lib.cpv_verify_tree(self.h, ctypes.c_void_p(self._tok.data_ptr()), par, t, nz,
                                                     ctypes.byref(out)))
        V, E = self.model.hp.n_vocab, self.model.hp.n_embd
        preds = _device_view(out.preds_dev, t, torch.int32, self.ctx.torch_device).cpu().tolist()
        logits = hidden = None
        if want_logits:
            logits = _device_view(out.logits_dev, t * V, torch.float32, self.ctx.torch_device).view(t, V).clone()
            hidden = _device_view(out.hidden_dev, t * E, torch.float32, self.ctx.torch_device).view(t, E).clone()
        return FusedOut(preds, [], [], logits, hidden)

    def accept_round(self, out, drafts, params, mode, noise=None, hist=None, key=0, round=0):
        """Decide a verified round on the device (cpv_spec_accept over the
        round's logits, out.logits [t][V] with t = len(drafts) + 1): returns
        (the accepted drafts then the next token, the number accepted).
        Uniforms are Philox4x64-10 with key (key, 0), counter (0, j, role,
        round);
        `noise` ([t][V], T-scaled gumbel) for the gumbel mode; `hist` the
        penalty window, oldest first."""
        t, V = out.logits.shape
        dev = self.ctx.torch_device
        dr = torch.tensor(list(drafts), dtype=torch.int32, device=dev).view(1, len(drafts))
        h = None if not hist else torch.tensor(list(hist), dtype=torch.int32, device=dev).view(1, -1)
        nz = None if noise is None else _as_device(noise, dev).view(1, t, V)
        tok, n = self.ctx.spec_accept(out.logits.view(1, t, V), dr, params, mode, noise=nz, hist=h,
                                      philox_seed=int(key), philox_round=int(round))
        n = int(n.cpu()[0])
        return tok[0, :n + 1].cpu().tolist(), n

    def commit_branch(self, path):
        """Keep the root-to-node path `path` (node indices) of the last tree
        verify as context rows; the other nodes are dropped."""
        n = len(path)
        arr = (ctypes.c_int32 * max(n, 1))(*[int(v) for v in path])
        self.ctx._check(self.ctx.lib.cpv_session_commit_branch(self.h, arr, n))

    def free(self):
        if self.h:
            self.ctx.lib.cpv_session_free(self.h)
            self.h = None


def _as_device(x, device):
    """A float32 cuda tensor of x (numpy or torch), contiguous."""
    if not isinstance(x, torch.Tensor):
        x = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return x.to(device=device, dtype=torch.float32).contiguous()


def _device_view(ptr, n, dtype, device):
    """A torch view of library-owned device memory (valid until the next call)."""
    class _Arr:
        __cuda_array_interface__ = {
            "shape": (n,), "typestr": {torch.int32: "<i4", torch.float32: "<f4"}[dtype],
            "data": (ptr, False), "version": 3, "strides": None,
        }
    return torch.as_tensor(_Arr(), device=device)


@dataclass
class FusedStats:
    accepted: int
    proposed: int
    rounds: int
    prefill_s: float = 0.0
    decode_s: float = 0.0
    redraft_rounds: int = 0     # rounds after which the drafts were re-drafted (sampled loop)
    redraft_links: int = 0      # standalone draft links run (each advances mtp_past)


def fused_generate(session, prompt, n_gen, depth, tail=64, bulk=512, timer=None, drafter=None):
    """cmd_fused (crates/codpiece-cli/src/main.rs:643-931) at a fixed depth with
    greedy acceptance; the seeded model has no tokenizer, so no EOS stop.
    drafter(committed, chain_drafts) -> drafts, when given, supplies each
    round's drafts instead of the MTP chain (an external drafter, as the
    engine's verify-only rounds take DFlash drafts, engine.rs:2291-2293); the
    chain is still computed at `depth`.  depth 0 with no drafter is plain
    greedy decoding, one token per round.
    When n_gen is reached inside a round's accepted drafts the loop ends
    there, before the round's rewind, as the reference's does (`break
    'outer`, main.rs:883-887): the session's n_past then still counts that
    round's unused rows, so a caller that reuses the session sets its
    positions first.
    Returns (committed tokens, FusedStats)."""
    import time
    t0 = time.perf_counter()
    split = max(0, len(prompt) - tail)
    bulk = min(bulk, getattr(session, "max_batch", bulk))
    for c in range(0, split, bulk):
        session.prefill(prompt[c:min(split, c + bulk)])
    out = session.step_fused_cached(prompt[split:], depth)
    n_past, mtp_past = session.pos
    session.set_pos(n_past, mtp_past + len(out.preds))
    last = len(out.preds) - 1
    committed = [out.preds[last]]
    drafts = [out.chain[l][last] for l in range(depth)]
    if drafter is not None:
        drafts = list(drafter(committed, drafts))
    t1 = time.perf_counter()
    accepted = proposed = rounds = 0
    while len(committed) < n_gen:
        batch = [committed[-1]] + drafts
        out = session.step_fused_cached(batch, depth)
        rounds += 1
        proposed += len(drafts)
        keep = 0
        while keep < len(drafts) and out.preds[keep] == drafts[keep]:
            keep += 1
        accepted += keep
        done = False
        for d in drafts[:keep]:
            committed.append(d)
            if len(committed) >= n_gen:
                done = True
                break
        if done:
            break
        committed.append(out.preds[keep])
        drafts = [out.chain[l][keep] for l in range(depth)]
        if drafter is not None:
            drafts = list(drafter(committed, drafts))
        over = len(batch) - (keep + 1)
        n_past, mtp_past = session.pos
        session.set_pos(n_past - over, mtp_past + keep + 1)
    t2 = time.perf_counter()
    return committed, FusedStats(accepted, proposed, rounds, t1 - t0, t2 - t1)


def _penalties_on(p):
    return p.penalty_last_n > 0 and (p.penalty_repeat != 1.0 or p.penalty_freq != 0.0 or p.penalty_present != 0.0)


def redraft(session, hidden, token, n_links, p_min, give_back=False):
    """Draft links from `hidden` and `token` at rope position n_past, chained
    on the drafts and the links' own hiddens, until n_links or the gate stops
    one (engine.rs:2584-2625; the CLI spec path, crates/codpiece-cli/src/
    main.rs:1052-1089, also gives the stopped link's MTP row back).  Returns
    (drafts, links run)."""
    drafts = []
    pos = session.pos[0]
    h, tok = hidden, token
    links = 0
    for _ in range(n_links):
        r = session.mtp_draft(h, tok, pos, p_min)
        links += 1
        if not r.keep:
            if give_back:
                n_past, mtp_past = session.pos
                session.set_pos(n_past, mtp_past - 1)
            break
        drafts.append(r.draft)
        tok, h = r.draft, r.hidden_ptr
        pos += 1
    return drafts, links


def spec_generate(session, prompt, n_gen, n_spec=1, p_min=0.75, tail=64, bulk=512):
    """cmd_spec (crates/codpiece-cli/src/main.rs:956-1180) without the context
    oracle (--oracle 0, its default) and without EOS: the prompt through the
    trunk (bulk prefill, then the last `tail` tokens as a verify-only round
    for the last row's argmax and hidden), then rounds of: up to n_spec
    standalone draft links from the last committed token and hidden, stopped
    (and the link's MTP row given back) at the first below p_min; a
    verify-only round of [last] + drafts; greedy acceptance; the rejected
    drafts rewound from n_past and mtp_past.  Returns (committed, FusedStats)."""
    import time
    t0 = time.perf_counter()
    split = max(0, len(prompt) - tail)
    bulk = min(bulk, getattr(session, "max_batch", bulk))
    for c in range(0, split, bulk):
        session.prefill(prompt[c:min(split, c + bulk)])
    out = session.step_fused_cached(prompt[split:], 0, want_logits=True)
    at = len(out.preds) - 1
    committed = [out.preds[at]]
    hidden = out.hidden[at]
    t1 = time.perf_counter()
    accepted = proposed = rounds = links = 0
    while len(committed) < n_gen:
        last = committed[-1]
        drafts, nl = redraft(session, hidden, last, n_spec, p_min, give_back=True)
        links += nl
        batch = [last] + drafts
        out = session.step_fused_cached(batch, 0, want_logits=True)
        rounds += 1
        proposed += len(drafts)
        keep = 0
        while keep < len(drafts) and out.preds[keep] == drafts[keep]:
            keep += 1
        accepted += keep
        done = False
        for d in drafts[:keep]:
            committed.append(d)
            if len(committed) >= n_gen:
                done = True
                break
        if done:
            break
        committed.append(out.preds[keep])
        hidden = out.hidden[keep]
        extra = len(drafts) - keep
        if extra:
            n_past, mtp_past = session.pos
            session.set_pos(n_past - extra, mtp_past - extra)
    t2 = time.perf_counter()
    return committed, FusedStats(accepted, proposed, rounds, t1 - t0, t2 - t1, 0, links)


def mtp_probe(session, prompt, n_gen, tail=64, bulk=512):
    """cmd_mtp_probe (crates/codpiece-cli/src/main.rs:1205-1293) without EOS:
    plain greedy decoding one token per verify-only step, with one standalone
    draft link per step predicting the token after next.  Returns (the greedy
    stream, hits, total): how often the link's draft was the next token."""
    split = max(0, len(prompt) - tail)
    bulk = min(bulk, getattr(session, "max_batch", bulk))
    for c in range(0, split, bulk):
        session.prefill(prompt[c:min(split, c + bulk)])
    out = session.step_fused_cached(prompt[split:], 0, want_logits=True)
    at = len(out.preds) - 1
    nxt, hidden = out.preds[at], out.hidden[at]
    stream, drafted, hits, total = [nxt], None, 0, 0
    for _ in range(n_gen):
        if drafted is not None:
            total += 1
            hits += int(drafted == nxt)
        drafted = session.mtp_draft(hidden, nxt, session.pos[0]).draft
        out = session.step_fused_cached([nxt], 0, want_logits=True)
        nxt, hidden = out.preds[0], out.hidden[0]
        stream.append(nxt)
    return stream, hits, total


def sampled_generate(session, prompt, n_gen, depth, params, mode=_lib.ACCEPT_REJECT, seed=0, tail=64, bulk=512,
                     noise=None, chain_pmin=0.0, drafter=None, redraft_depth=3, redraft_pmin=0.75):
    """The engine's sampled speculative loop for one request (crates/codpiece-
    server/src/engine.rs), at a fixed draft depth, without EOS, stop strings,
    JSON or forced tokens:
      * the prompt seeds the penalty window (sampler.accept_all, :1764); all
        but the last `tail` tokens are prefilled in `bulk` chunks (:1922-1953);
      * the tail runs as a fused round; the first token is a draw from the
        distribution at the last position, and the drafts are the chain there
        (:1958-2012, :2039);
      * each round verifies [next] + drafts with the chain at `depth`
        (:2291-2305) and decides them on the device (cpv_spec_accept):
        REJECT accepts draft j with probability p(x_j), else draws the
        replacement excluding x_j (:2351-2359); GUMBEL accepts a draft iff it
        is the gumbel-coupled sample (:2336-2349); the next token is the
        replacement, or else a draw at the first unverified position (:2400-
        2461); every committed token enters the penalty window (:2368, :2497);
      * the next drafts are the chain at n_keep, cut at the first link whose
        confidence is below chain_pmin (:2508-2517), and dropped when the next
        token is not the trunk's argmax there (:2527-2529); the rejected rows
        are rewound (:2533-2540);
      * when no draft is left, up to redraft_depth standalone draft links run
        from the trunk's hidden at n_keep and the next token, at rope position
        n_past, each kept while its softmax peak is at least redraft_pmin
        (the post-commit re-draft, :2584-2625; the engine's defaults,
        CODPIECE_REDRAFT = 3 and CODPIECE_REDRAFT_PMIN = 0.75, :2162-2185),
        cut to `depth`.  Every link run advances mtp_past, the stopped one
        included.  redraft_depth 0 turns it off; an external drafter (the
        engine's DFlash mode) has none.
    Randomness is explicit: the reference's sequential xoshiro stream becomes
    Philox4x64-10 uniforms by role, round r (the tail round is 0) using key
    (seed, 0) with counter (0, j, role, r).  In GUMBEL mode noise(r, rows)
    supplies round r's T-scaled gumbel noise [rows][V] (the engine's noise
    thread, :2080-2118): the verify argmaxes logits + noise in the graph, and
    the acceptance couples on the same noise.  drafter(committed, drafts), when
    given, replaces each round's drafts after those rules (an external
    drafter, as fused_generate takes).  As in fused_generate (and the
    engine's `break 'outer`), a run that ends inside a round's accepted
    drafts leaves that round unrewound.  Returns (committed tokens,
    FusedStats)."""
    import time
    if mode == _lib.ACCEPT_GUMBEL and noise is None:
        raise ValueError("sampled_generate: the gumbel mode needs a noise source")
    t0 = time.perf_counter()
    window = deque(maxlen=params.penalty_last_n) if _penalties_on(params) else None

    def seen(tok):
        if window is not None:
            window.append(int(tok))

    def hist():
        return list(window) if window else None

    for tok in prompt:
        seen(tok)
    split = max(0, len(prompt) - tail)
    bulk = min(bulk, getattr(session, "max_batch", bulk))
    for c in range(0, split, bulk):
        session.prefill(prompt[c:min(split, c + bulk)])
    out = session.step_fused_cached(prompt[split:], depth, want_logits=True)
    n_past, mtp_past = session.pos
    session.set_pos(n_past, mtp_past + len(out.preds))
    at = len(out.preds) - 1
    first = FusedOut(out.preds[at:], [], [], out.logits[at:at + 1], None)
    toks, _ = session.accept_round(first, [], params, _lib.ACCEPT_REJECT, hist=hist(), key=seed)
    nxt = toks[0]
    seen(nxt)
    committed = [nxt]
    drafts = [out.chain[l][at] for l in range(depth)]
    if drafter is not None:
        drafts = list(drafter(committed, drafts))
    t1 = time.perf_counter()
    accepted = proposed = rounds = re_rounds = re_links = 0
    while len(committed) < n_gen:
        rounds += 1
        batch = [nxt] + drafts
        nz = noise(rounds, len(batch)) if mode == _lib.ACCEPT_GUMBEL else None
        out = session.step_fused_cached(batch, depth, want_logits=True, noise=nz)
        proposed += len(drafts)
        toks, keep = session.accept_round(out, drafts, params, mode, noise=nz, hist=hist(), key=seed, round=rounds)
        accepted += keep
        done = False
        for d in drafts[:keep]:
            seen(d)
            committed.append(d)
            if len(committed) >= n_gen:
                done = True
                break
        if done:
            break
        nxt = toks[keep]
        seen(nxt)
        committed.append(nxt)
        drafts = []
        for l in range(depth):
            if out.conf[l][keep] < chain_pmin:
                break
            drafts.append(out.chain[l][keep])
        if nxt != out.preds[keep]:
            drafts = []
        if drafter is not None:
            drafts = list(drafter(committed, drafts))
        over = len(batch) - (keep + 1)
        n_past, mtp_past = session.pos
        session.set_pos(n_past - over, mtp_past + keep + 1)
        if not drafts and redraft_depth > 0 and drafter is None:
            drafts, nl = redraft(session, out.hidden[keep], nxt, redraft_depth, redraft_pmin)
            drafts = drafts[:depth]
            re_rounds += 1
            re_links += nl
    t2 = time.perf_counter()
    return committed, FusedStats(accepted, proposed, rounds, t1 - t0, t2 - t1, re_rounds, re_links)


__all__ = ["Model", "Session", "FusedOut", "FusedStats", "DraftResult", "make_hparams", "fused_generate",
           "sampled_generate", "spec_generate", "mtp_probe", "redraft", "CpvError"]
