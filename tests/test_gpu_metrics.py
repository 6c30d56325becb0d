"""Runtime metrics from the engine (through the C ABI): moert_generate with an attached publisher fills the
reference monitor's snapshot (rust/moe-monitor/src/snapshot.rs) from the device counters, and the per-token counters
of the expert cache add up to its totals."""
import json

import numpy as np
import pytest

import moert

pytestmark = pytest.mark.gpu

TINY8 = dict(hidden=256, inter=128, layers=3, heads=4, kv_heads=2, head_dim=64, vocab=97, experts=8, top_k=2)


def say(msg):
    print(f"[case] {msg}", flush=True)


def _model():
    cfg = moert.Config(**TINY8)
    return cfg, moert.SynthModel(cfg, seed=13, wdtype=moert.Q4_0, embed_dtype=moert.F32, std=0.1, zipf_s=1.1)


@pytest.mark.parametrize("interval_ms", [0, 500])
def test_generate_publishes_the_request_and_the_cache_totals(gpu, tmp_path, interval_ms):
    """A cached model generating 5 prompt + 40 new tokens with a publisher attached: the same tokens as without one;
    the final snapshot is idle, with the request (prompt / output tokens, rates, status), the context used, the pool
    size and the cumulative hits and copies equal to moert_cache_stats; the per-position, per-layer counters of
    moert_cache_token_counts add up to the same totals."""
    cfg, m = _model()
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 5)
    plain = moert.GpuModel(m, 64, attn_splits=4, cache_slots=6)
    want = plain.generate(prompt, 40)
    plain.close()
    g = moert.GpuModel(m, 64, attn_splits=4, cache_slots=6)
    path = tmp_path / "metrics.json"
    mx = moert.Metrics(path)
    say(f"metrics attach interval={interval_ms}")
    g.attach_metrics(mx, interval_ms)
    kind, s = moert.read_metrics(path)
    assert kind == "live" and s["state"] == {"kind": "idle"}
    assert s["model"] == {"name": "granite-moe", "layers": 3, "experts": 8, "experts_per_tok": 2}
    assert s["settings"]["expert pool slots"] == "6 of 24"
    say("metrics generate")
    got = g.generate(prompt, 40)
    assert np.array_equal(got, want)
    kind, s = moert.read_metrics(path)
    assert kind == "live" and s["state"] == {"kind": "idle"}
    hits, copies = g.cache_stats()
    c = s["cache"]
    assert (c["total_hits"], c["total_copies"], c["total_cpu"]) == (hits, copies, 0)
    assert c["slots_total"] == 6 and 0 < c["slots_resident"] <= 6
    assert c["slots_loading"] == 0 and c["copies_inflight"] == 0
    assert 0.0 <= c["hit_frac"] <= 1.0 and abs(c["hit_frac"] + c["copy_frac"] - 1.0) < 1e-12
    assert s["context"] == {"used": 44, "max": 64}
    r = s["requests"][0]
    assert (r["prompt_tokens"], r["output_tokens"], r["status"]) == (5, 40, "ok")
    assert r["decode_tok_s"] > 0 and r["prefill_tok_s"] > 0
    assert s["speed"]["decode_last"] == r["decode_tok_s"]
    assert s["window"]["ms_per_token"] > 0 and 0.0 <= s["window"]["gpu_wait_frac"] <= 1.0
    assert "40 new tokens" in s["events"][-1]["message"]
    counts = g.cache_token_counts(0, 44)
    assert counts[:, :, 0].sum() == hits and counts[:, :, 1].sum() == copies
    assert (counts[:, :, 0] + counts[:, :, 1] == cfg.top_k).all()
    g.attach_metrics(None)
    g.close()
    mx.close()


def test_resident_model_reports_every_expert_resident_and_errors_as_error_state(gpu, tmp_path):
    """A resident model publishes hit_frac 1 over all layers x experts (as the reference does for its resident
    runs); a refused generate call leaves the error state, a failed request and an error event."""
    cfg, m = _model()
    g = moert.GpuModel(m, 64, attn_splits=4)
    path = tmp_path / "metrics.json"
    mx = moert.Metrics(path)
    g.attach_metrics(mx, 0)
    g.generate([1, 2, 3], 4)
    s = json.loads(path.read_text())
    assert s["cache"]["slots_total"] == s["cache"]["slots_resident"] == 24 and s["cache"]["hit_frac"] == 1.0
    assert s["requests"][0]["output_tokens"] == 4
    say("metrics refused generate")
    with pytest.raises(moert.MoertError):
        g.generate([1, 2, 3], 60)  # 6 + 62 positions > 64
    s = json.loads(path.read_text())
    assert s["state"]["kind"] == "error" and "KV cache full" in s["state"]["message"]
    assert s["requests"][0]["status"] == "erro" and s["events"][-1]["level"] == "erro"
    g.generate([4], 2)  # the model still works after a refused call
    assert json.loads(path.read_text())["state"] == {"kind": "idle"}
    g.attach_metrics(None)
    g.close()
    mx.close()
