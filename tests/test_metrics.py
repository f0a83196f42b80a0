"""Serving metrics of the attention path (the reference's /metrics lines,
app/api/server.py:275-310, plus attention latency and GB/s)."""

import pytest
import torch

from helpers import pkg

metrics = pkg("metrics")
manager_mod = pkg("memory.manager")
sequence_mod = pkg("engine.request")


class FakeEvent:
    def __init__(self, t, done=True):
        self.t, self.done = t, done

    def query(self):
        return self.done

    def elapsed_time(self, other):
        return other.t - self.t


def test_aggregates_completed_calls_only():
    m = metrics.AttentionMetrics(ema=0.5)
    m.add(FakeEvent(0.0), FakeEvent(2.0), nbytes=16_000_000_000, tokens=100)  # 2 ms at 8 TB/s
    m.add(FakeEvent(0.0), FakeEvent(1.0, done=False), nbytes=10, tokens=1)
    assert m.poll() == 1 and m.pending == 1
    assert m.calls == 1 and m.last_ms == 2.0 and m.avg_ms == 2.0
    assert abs(m.last_gbps - 8000.0) < 1e-6
    text = dict(line.split() for line in m.lines())
    assert float(text["paged_attention_hbm_peak_fraction"]) == pytest.approx(1.0)
    assert float(text["paged_attention_tokens_per_second"]) == pytest.approx(100 / 2e-3)
    assert text["paged_attention_pending_events"] == "1"


def test_pending_queue_is_bounded():
    m = metrics.AttentionMetrics(max_pending=2)
    for _ in range(5):
        m.add(FakeEvent(0.0, done=False), FakeEvent(1.0, done=False), 1, 1)
    assert m.pending == 2 and m.dropped == 3


def test_step_bytes_matches_the_decode_formula():
    # 2 sequences, contexts 17 and 32, H_q 8 / H_kv 2, D 64, bf16, bs 16
    got = metrics.step_bytes([17, 32], 2, 8, 2, 64, 2, 16)
    kv = (17 + 32) * 2 * 2 * 64 * 2
    qo = 2 * 8 * 64 * 2 * 2
    assert got == kv + qo + (2 + 2) * 4 + 2 * 4


def test_metrics_text_has_the_reference_lines(monkeypatch):
    monkeypatch.delenv("LLM_PAGED_METRICS", raising=False)
    metrics.disable()
    mgr = manager_mod.PagedKVCacheManager(total_blocks=10, block_size=4, num_heads=2, head_dim=8, device="cpu")
    seq = sequence_mod.Request(seq_id=1, prompt_token_ids=[1, 2, 3, 4, 5])
    mgr.allocate_prefix_blocks(seq)
    text = metrics.metrics_text(mgr)
    lines = dict(line.split() for line in text.strip().splitlines())
    assert float(lines["kv_cache_free_pages_ratio"]) == pytest.approx(8 / 10)
    assert lines["kv_cache_active_streams"] == "0" and lines["kv_cache_preemptions_total"] == "0"
    assert "paged_attention_calls_total" not in lines
    metrics.enable()
    assert "paged_attention_calls_total 0" in metrics.metrics_text(mgr)
    metrics.disable()


@pytest.mark.gpu
def test_native_backend_records_attention(device):
    transformers = pytest.importorskip("transformers")
    paged_attention = pkg("model.paged_attention")
    backends = pkg("model.attention_backends")
    cfg = transformers.LlamaConfig(vocab_size=128, hidden_size=512, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=1024)
    torch.manual_seed(0)
    model = transformers.LlamaForCausalLM(cfg).to(device=device, dtype=torch.bfloat16).eval()
    store = manager_mod.PagedKVCacheManager.from_model_config(cfg, total_blocks=64, block_size=16,
                                                              dtype=torch.bfloat16, device=device)
    paged_attention.register_paged_attention(model)
    old = paged_attention._BACKEND
    paged_attention._BACKEND = backends.NativePagedBackend()
    rec = metrics.enable()
    try:
        seq = sequence_mod.Request(seq_id=1, prompt_token_ids=list(range(40)))
        store.allocate_prefix_blocks(seq)
        ctx = paged_attention.PagedStepContext(store, [seq], [0], [40])
        with torch.inference_mode():
            paged_attention.run_paged_forward(model, ctx, torch.arange(40, device=device)[None])
        torch.cuda.synchronize()
        assert rec.poll() == 2  # one call per layer
        assert rec.calls == 2 and rec.last_ms > 0 and rec.total_bytes > 0
        assert "paged_attention_calls_total 2" in metrics.metrics_text(store)
    finally:
        metrics.disable()
        paged_attention._BACKEND = old
