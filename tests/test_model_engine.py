"""End-to-end: a transformers Llama GQA model served through the paged hook.

Mirrors the reference's model-level checks (tests/correctness/
test_paged_attention.py:48-84: paged greedy generation equals the model's own
generation) on an offline, random-init tiny Llama built from a config with a
fixed seed, as tests/fuzz/test_allocator_scheduler_fuzzing.py:309-323 does.
No checkpoint is downloaded.

Every engine step is teacher-forced on the same token stream as a plain
no-cache forward of the whole sequence, and the step's logits are compared
with that forward's logits at the same positions; greedy tokens are compared
where the top-2 margin exceeds the tolerance (a random model has near-ties).
An fp32 model is held to an absolute tolerance.  A bf16 model is compared
with an fp32 copy of itself: over the rows of a step, its largest and its
mean error may be at most 1.5x (+0.02 / +0.01) those of the model's own bf16
SDPA forward over the same rows.

CPU tests run the reference's inline SDPA path over a CPU store.  GPU tests
install the HIP backend (decode split-K + MFMA prefill, packing and K/V write
on the device) over an HBM store, and run ragged multi-sequence and mixed
prefill + decode steps.
"""

import copy

import pytest
import torch

from helpers import pkg

transformers = pytest.importorskip("transformers")

paged_attention = pkg("model.paged_attention")
backends = pkg("model.attention_backends")
manager_mod = pkg("memory.manager")
sequence_mod = pkg("engine.request")

BLOCK_SIZE = 16


def tiny_llama(dtype, device, seed=0, head_dim=64, layers=2, heads=8, kv_heads=2):
    cfg = transformers.LlamaConfig(
        vocab_size=512,
        hidden_size=heads * head_dim,
        intermediate_size=1024,
        num_hidden_layers=layers,
        num_attention_heads=heads,
        num_key_value_heads=kv_heads,
        max_position_embeddings=4096,
        initializer_range=0.08,
    )
    torch.manual_seed(seed)
    model = transformers.LlamaForCausalLM(cfg).to(device=device, dtype=dtype)
    model.eval()
    return model


def reference_logits(model, ids, device):
    """Logits of a plain forward of the whole sequence (model's own attention)."""
    cfg_impl = model.config._attn_implementation
    model.config._attn_implementation = "sdpa"
    try:
        with torch.inference_mode():
            out = model(torch.tensor([ids], device=device), use_cache=False).logits[0].float()
    finally:
        model.config._attn_implementation = cfg_impl
    return out


class Reference:
    """Reference logits of a sequence and the error bound a paged step must meet."""

    def __init__(self, model, device, tol):
        self.model, self.device, self.tol = model, device, tol
        self.exact = None
        if model.dtype != torch.float32:
            self.exact = copy.deepcopy(model).float()

    def __call__(self, ids):
        """(logits to compare with, per-row error of the model's own forward or
        None when the absolute tolerance applies)."""
        own = reference_logits(self.model, ids, self.device)
        if self.exact is None:
            return own, None
        exact = reference_logits(self.exact, ids, self.device)
        return exact, (own - exact).abs()


class Stepper:
    """Teacher-forced steps through the paged hook: one flat forward per step
    over any mix of prefill chunks and decodes, on token streams fixed in
    advance (the product engine, which feeds back its own tokens, is tested
    below)."""

    def __init__(self, model, device, total_blocks=256):
        self.model = model
        self.device = device
        self.store = manager_mod.PagedKVCacheManager.from_model_config(
            model.config, total_blocks=total_blocks, block_size=BLOCK_SIZE, dtype=model.dtype, device=device)
        paged_attention.register_paged_attention(model, backend=paged_attention._BACKEND)
        self.next_id = 1

    def add(self, prompt):
        seq = sequence_mod.Request(seq_id=self.next_id, prompt_token_ids=list(prompt))
        self.next_id += 1
        self.store.allocate_prefix_blocks(seq)
        return seq

    def step(self, entries):
        """entries: (seq, start, tokens) -> per-entry logits [len(tokens), V]."""
        seqs, starts, toks = [], [], []
        for seq, start, tokens in entries:
            while seq.block_table.get_tokens_count() < start + len(tokens):
                self.store.allocate_slot_for_next_token(seq)
            seqs.append(seq)
            starts.append(start)
            toks.append(list(tokens))
        ctx = paged_attention.PagedStepContext(self.store, seqs, starts, [len(t) for t in toks])
        flat = torch.tensor([[t for ts in toks for t in ts]], dtype=torch.long, device=self.device)
        with torch.inference_mode():
            logits = paged_attention.run_paged_forward(self.model, ctx, flat)[0].float()
        out, off = [], 0
        for ts in toks:
            out.append(logits[off : off + len(ts)])
            off += len(ts)
        return out


def check_logits(got, ref, tol):
    want, own_err = ref
    err = (got - want).abs()
    if own_err is None:
        bound = tol
        assert err.max().item() <= bound, f"max |logit diff| {err.max().item():.3e} > {bound:.1e}"
    else:
        bound = 1.5 * own_err.max().item() + 0.02
        assert err.max().item() <= bound, (
            f"max |logit diff| {err.max().item():.3e} > 1.5 x bf16 SDPA's {own_err.max().item():.3e} + 0.02")
        assert err.mean().item() <= 1.5 * own_err.mean().item() + 0.01, (
            f"mean |logit diff| {err.mean().item():.3e} vs bf16 SDPA's {own_err.mean().item():.3e}")
    top2 = torch.topk(want, 2, dim=-1).values
    decisive = (top2[:, 0] - top2[:, 1]) > 4 * bound
    assert torch.equal(got.argmax(-1)[decisive], want.argmax(-1)[decisive])


def _rows(ref, a, b):
    return ref[0][a:b], (None if ref[1] is None else ref[1][a:b])


def run_scenario(model, device, tol, prompts, decode_steps, late_prompt=None):
    torch.manual_seed(123)
    vocab = model.config.vocab_size
    streams = [list(p) + torch.randint(0, vocab, (decode_steps,)).tolist() for p in prompts]
    eng = Stepper(model, device)
    reference = Reference(model, device, tol)
    seqs = [eng.add(p) for p in prompts]
    # step 0: all prompts prefilled together (ragged)
    outs = eng.step([(s, 0, p) for s, p in zip(seqs, prompts)])
    refs = [reference(st) for st in streams]
    for o, r, p in zip(outs, refs, prompts):
        check_logits(o, _rows(r, 0, len(p)), tol)
    late = None
    for k in range(decode_steps):
        entries = [(s, len(p) + k, [st[len(p) + k]]) for s, p, st in zip(seqs, prompts, streams)
                   if len(p) + k < len(st)]
        if late_prompt is not None and k == decode_steps // 2:
            late = eng.add(late_prompt)
            entries.append((late, 0, list(late_prompt)))  # a prefill mixed with decodes
        outs = eng.step(entries)
        for (s, pos, tok), o in zip(entries, outs):
            if s is late:
                check_logits(o, reference(list(late_prompt)), tol)
            else:
                i = seqs.index(s)
                check_logits(o, _rows(refs[i], pos, pos + 1), tol)
    return eng


# ---------------------------------------------------------------------------
# CPU: the reference's inline path over a CPU store


def test_cpu_paged_generation_matches_model(monkeypatch):
    monkeypatch.setattr(paged_attention, "_BACKEND", None)
    model = tiny_llama(torch.float32, "cpu")
    run_scenario(model, "cpu", 1e-4, prompts=[[5, 9, 2, 7, 1], [3, 3, 8]], decode_steps=4)


def test_cpu_cache_holds_history_for_every_layer(monkeypatch):
    # tests/correctness/test_paged_attention.py:87-119
    monkeypatch.setattr(paged_attention, "_BACKEND", None)
    model = tiny_llama(torch.float32, "cpu", layers=3)
    eng = Stepper(model, "cpu", total_blocks=32)
    prompt = list(range(1, 20))
    seq = eng.add(prompt)
    eng.step([(seq, 0, prompt)])
    assert eng.store.key_cache.shape == (3, 32, BLOCK_SIZE, 2, 64)
    empty = paged_attention.PagedStepContext(eng.store, [seq], [0], [0])
    assert empty.gather_slots.numel() == 0
    full = paged_attention.PagedStepContext(eng.store, [seq], [0], [len(prompt)])
    for layer in range(3):
        keys = eng.store.gather_layer_keys(layer, full.gather_slots)
        assert keys.shape == (len(prompt), 2, 64)
        assert torch.isfinite(keys).all() and keys.abs().sum() > 0


# ---------------------------------------------------------------------------
# GPU: the HIP backend installed behind the same hook


@pytest.fixture
def native(monkeypatch):
    backend = backends.select_backend("native")
    assert isinstance(backend, backends.NativePagedBackend)
    monkeypatch.setattr(paged_attention, "_BACKEND", backend)
    return backend


class _NoFallback(backends.TorchSdpBackend):
    def attend(self, *args, **kwargs):
        raise AssertionError("the HIP backend refused a step of a GPU store")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-3), (torch.bfloat16, None)])
def test_gpu_engine_matches_model(native, monkeypatch, dtype, tol):
    monkeypatch.setattr(paged_attention, "_FALLBACK_BACKEND", _NoFallback())
    model = tiny_llama(dtype, "cuda")
    prompts = [list(range(3, 40)), [7, 1, 4], list(range(100, 300)), [11] * 70]
    run_scenario(model, "cuda", tol, prompts, decode_steps=6, late_prompt=list(range(50, 95)))


@pytest.mark.gpu
def test_gpu_engine_long_context_split_k(native, monkeypatch):
    """A prompt longer than the decode partition (split-K + merge path)."""
    monkeypatch.setattr(paged_attention, "_FALLBACK_BACKEND", _NoFallback())
    model = tiny_llama(torch.bfloat16, "cuda", head_dim=128)
    torch.manual_seed(7)
    prompt = torch.randint(0, 512, (2500,)).tolist()
    run_scenario(model, "cuda", None, [prompt, prompt[:300]], decode_steps=3)


@pytest.mark.gpu
def test_gpu_engine_smollm_head_shape(native, monkeypatch):
    """9 query heads over 3 KV heads of 64 (SmolLM-135M's attention shape, the
    reference's test model): a group of three on the HIP decode and prefill."""
    monkeypatch.setattr(paged_attention, "_FALLBACK_BACKEND", _NoFallback())
    model = tiny_llama(torch.bfloat16, "cuda", heads=9, kv_heads=3)
    prompts = [list(range(3, 60)), [7, 1, 4], list(range(100, 230))]
    run_scenario(model, "cuda", None, prompts, decode_steps=4, late_prompt=list(range(50, 90)))


# ---------------------------------------------------------------------------
# The product engine: one forward per step, GPU argmax, HIP backend installed


engine_mod = pkg("engine.llm_engine")


def _generate(model, prompt, n, device):
    """Greedy continuation by the model's own generate() (SDPA, its own cache)."""
    impl = model.config._attn_implementation
    model.config._attn_implementation = "sdpa"
    try:
        with torch.inference_mode():
            ids = torch.tensor([prompt], device=device)
            out = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=n, do_sample=False,
                                 pad_token_id=0)
    finally:
        model.config._attn_implementation = impl
    return out[0, len(prompt):].tolist()


def run_engine(model, device, prompts, late_prompt, max_tokens, total_blocks=256, block_size=BLOCK_SIZE,
               scheduler=None, total_cpu_blocks=32):
    """Serve ``prompts`` (and ``late_prompt``, added after the second step so
    that a prefill shares a step with decodes) through LLMEngine.step().
    ``max_tokens`` is one limit for all or one per prompt (late prompt last);
    ``scheduler`` builds the scheduler from the store (default: first come,
    first served).  Returns (requests, steps, store, scheduler)."""
    from fcfs import FcfsScheduler

    store = manager_mod.PagedKVCacheManager.from_model_config(
        model.config, total_blocks=total_blocks, block_size=block_size, dtype=model.dtype, device=device,
        total_cpu_blocks=total_cpu_blocks)
    sched = (scheduler or FcfsScheduler)(store)
    engine = engine_mod.LLMEngine(store, sched, model=model)
    limits = list(max_tokens) if isinstance(max_tokens, (list, tuple)) else \
        [max_tokens] * (len(prompts) + (late_prompt is not None))
    calls = {"n": 0}
    forward = model.forward

    def counted(*args, **kwargs):
        calls["n"] += 1
        return forward(*args, **kwargs)

    model.forward = counted
    try:
        eos = model.config.eos_token_id  # generate() stops there too
        reqs = [engine.add_request(p, max_tokens=n, eos_token_id=eos) for p, n in zip(prompts, limits)]
        steps = mixed = idle = 0
        late = None
        while engine.has_unfinished_requests():
            if steps == 2 and late_prompt is not None:
                late = engine.add_request(late_prompt, max_tokens=limits[-1], eos_token_id=eos)
            before = calls["n"]
            result = engine.step()
            steps += 1
            if calls["n"] == before:  # nothing was runnable (a request is swapped out)
                idle += 1
                assert idle < 8, "the scheduler stalled"
                continue
            assert calls["n"] == before + 1, "one forward per step"
            if late is not None and late in result["running"] and len(late.output_token_ids) == 1:
                mixed += 1
    finally:
        model.forward = forward
    assert engine.forward_passes == steps - idle
    if late_prompt is not None:
        assert mixed == 1, "the late prompt was prefilled in a step with decodes"
        reqs.append(late)
    assert store.get_allocator().get_num_free_blocks() == total_blocks
    assert store.get_allocator().get_num_free_cpu_blocks() == total_cpu_blocks
    assert all(r.block_table is None for r in reqs)
    return reqs, steps, store, sched


def test_cpu_engine_greedy_matches_generate(monkeypatch):
    monkeypatch.setattr(paged_attention, "_BACKEND", None)
    model = tiny_llama(torch.float32, "cpu")
    prompts = [[5, 9, 2, 7, 1], [3, 3, 8], list(range(40, 75))]
    late = [11, 12, 13, 14]
    reqs, steps, _, _ = run_engine(model, "cpu", prompts, late, max_tokens=6)
    # the first prompts finish at step 6; the late one, prefilled at step 3, at step 8
    assert steps == 8
    for req, prompt in zip(reqs, prompts + [late]):
        assert req.output_token_ids == _generate(model, prompt, 6, "cpu"), req.seq_id


def _no_dense(monkeypatch):
    def no_dense(*args, **kwargs):
        raise AssertionError("dense SDPA ran on a GPU store")

    monkeypatch.setattr(backends, "dense_sdpa", no_dense)
    monkeypatch.setattr(backends.TorchSdpBackend, "attend", no_dense)


@pytest.mark.gpu
@pytest.mark.parametrize("block_size", [1, 4, 16, 32, 64])
def test_gpu_engine_greedy_matches_generate(monkeypatch, block_size):
    """The product engine on an HBM store with no backend installed beforehand:
    it installs the HIP backend itself, never runs dense SDPA, makes one
    forward per step, and its greedy tokens equal the model's own generate()
    (fp32 model: HIP decode and fp32 prefill kernels), at the block sizes of
    the reference's end-to-end sweep (tests/correctness/
    test_correctness_spec.py:70-142); the pool holds 4096 tokens at each."""
    monkeypatch.setattr(paged_attention, "_BACKEND", None)
    _no_dense(monkeypatch)
    model = tiny_llama(torch.float32, "cuda")
    prompts = [list(range(3, 40)), [7, 1, 4], list(range(100, 300)), [11] * 70]
    late = list(range(50, 95))
    reqs, *_ = run_engine(model, "cuda", prompts, late, max_tokens=12, total_blocks=4096 // block_size,
                          block_size=block_size)
    assert isinstance(paged_attention._BACKEND, backends.NativePagedBackend)
    for req, prompt in zip(reqs, prompts + [late]):
        assert req.output_token_ids == _generate(model, prompt, 12, "cuda"), req.seq_id


# Preempt and resume (tests/correctness/test_correctness_spec.py:236-259):
# greedy output must not change when the scheduler preempts.  Six requests
# with staggered limits, so requests finish at different steps and waiting
# ones are admitted into the rows they free.
PREEMPT_PROMPTS = [list(range(3, 40)), [7, 1, 4], list(range(100, 160)), [11] * 70, list(range(200, 221)),
                   [5, 9, 2, 7, 1, 8, 8]]
PREEMPT_LIMITS = [14, 9, 12, 6, 11, 16]


def _preempting(plan, **kw):
    from fcfs import PreemptingScheduler

    return lambda store: PreemptingScheduler(store, plan=plan, **kw)


def _check_preempted_run(model, device, reqs, sched):
    for req, prompt, n in zip(reqs, PREEMPT_PROMPTS, PREEMPT_LIMITS):
        assert req.output_token_ids == _generate(model, prompt, n, device), req.seq_id


def test_cpu_engine_preempt_recompute_matches_generate(monkeypatch):
    """Recompute preemption on a CPU store: forced at chosen steps (the
    request is re-admitted in the same step), and by running out of blocks
    in a pool too small for every request at once."""
    monkeypatch.setattr(paged_attention, "_BACKEND", None)
    model = tiny_llama(torch.float32, "cpu")
    plan = {3: [(1, "recompute")], 5: [(3, "recompute"), (2, "recompute")], 9: [(1, "recompute")]}
    reqs, _, _, sched = run_engine(model, "cpu", PREEMPT_PROMPTS, None, PREEMPT_LIMITS, total_blocks=14,
                                   block_size=8, scheduler=_preempting(plan))
    assert sched.preempted["recompute"] >= 3 and sched.preempted["oom"] >= 1, sched.preempted
    _check_preempted_run(model, "cpu", reqs, sched)


@pytest.mark.gpu
@pytest.mark.parametrize("block_size,total_blocks", [(16, 16), (16, 12), (4, 46)])
def test_gpu_engine_preempt_and_resume_matches_generate(monkeypatch, block_size, total_blocks):
    """The product engine on an HBM store with requests preempted mid-run,
    both ways: by recompute (blocks freed, re-prefilled from prompt and
    outputs through the HIP prefill) and by swap (blocks copied to the
    pinned host pool, the device blocks reused by others, copied back into
    fresh blocks two steps later, decoding on).  The pool is too small for
    every request at once, so requests also get preempted when blocks run
    out and wait for others to finish.  Every request's greedy tokens equal
    generate(); device and host blocks all return to the free lists."""
    monkeypatch.setattr(paged_attention, "_BACKEND", None)
    _no_dense(monkeypatch)
    model = tiny_llama(torch.float32, "cuda")
    plan = {2: [(1, "swap")], 3: [(3, "recompute")], 6: [(2, "swap"), (5, "recompute")], 8: [(1, "recompute")],
            10: [(6, "swap")]}
    reqs, _, store, sched = run_engine(model, "cuda", PREEMPT_PROMPTS, None, PREEMPT_LIMITS,
                                       total_blocks=total_blocks, block_size=block_size,
                                       scheduler=_preempting(plan), total_cpu_blocks=64)
    assert sched.preempted["swap"] >= 2 and sched.preempted["recompute"] >= 2, sched.preempted
    assert sched.preempted["oom"] >= 1, sched.preempted
    _check_preempted_run(model, "cuda", reqs, sched)


@pytest.mark.gpu
def test_gpu_engine_bf16_long_context(monkeypatch):
    """bf16 GQA heads of 128 with a 2500-token prompt (split-K decode): the
    engine's first token equals generate()'s, every step is one forward, and
    every later token whose top-2 margin is decisive (about one in ten on
    this random model) is the fp32 model's argmax on the engine's own prefix."""
    monkeypatch.setattr(paged_attention, "_BACKEND", None)
    monkeypatch.setattr(backends, "dense_sdpa", lambda *a, **k: (_ for _ in ()).throw(AssertionError("dense")))
    model = tiny_llama(torch.bfloat16, "cuda", head_dim=128)
    torch.manual_seed(7)
    prompt = torch.randint(0, 512, (2500,)).tolist()
    reference = Reference(model, "cuda", None)  # its fp32 copy is taken before the engine hooks the model
    reqs, *_ = run_engine(model, "cuda", [prompt, prompt[:300]], None, max_tokens=24, total_blocks=512)
    decisive_total = 0
    for req, p in zip(reqs, [prompt, prompt[:300]]):
        assert 1 <= len(req.output_token_ids) <= 24
        assert req.output_token_ids[0] == _generate(model, p, 1, "cuda")[0]
        # every generated token, teacher-forced on the engine's own outputs:
        # where the fp32 copy's top-2 margin is decisive against the model's
        # own bf16 error on that row, the engine's token is its argmax
        ids = p + req.output_token_ids
        exact, own = reference(ids)
        rows = slice(len(p) - 1, len(ids) - 1)
        want, err = exact[rows], own[rows]
        bound = 1.5 * err.max(dim=-1).values + 0.02
        top2 = torch.topk(want, 2, dim=-1).values
        decisive = (top2[:, 0] - top2[:, 1]) > 4 * bound
        got = torch.tensor(req.output_token_ids, device=want.device)
        assert torch.equal(got[decisive], want.argmax(-1)[decisive]), req.seq_id
        decisive_total += int(decisive.sum())
    assert decisive_total >= 1
