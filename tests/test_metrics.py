"""The runtime metrics publisher (host only): the JSON snapshot of the reference's monitor transport
(rust/moe-monitor/src/snapshot.rs), its atomic publication and the reader's four outcomes, after the reference's
monitor tests (rust/moe-monitor/tests/monitor.rs:41-83)."""
import json
import math
import os
import threading

import pytest

import moert

SNAPSHOT_KEYS = ["schema", "ts_ms", "pid", "started_ms", "model", "state", "speed", "context", "cache", "window",
                 "requests", "settings", "events"]
SECTION_KEYS = {
    "model": ["name", "layers", "experts", "experts_per_tok"],
    "speed": ["decode_now", "decode_last", "prefill_now", "prefill_request"],
    "context": ["used", "max"],
    "cache": ["slots_total", "slots_resident", "slots_loading", "hit_frac", "copy_frac", "cpu_frac", "copies_inflight",
              "h2d_gbs", "total_hits", "total_copies", "total_cpu"],
    "window": ["exposure_frac", "gpu_wait_frac", "ms_per_token"],
}


def demo(path):
    """The reference test's demo snapshot (monitor.rs:33-40)."""
    mx = moert.Metrics(path)
    mx.set_model("teste", 32, 40, 8)
    mx.set_state(moert.STATE_GENERATING, 120, 400)
    mx.set_cache(slots_total=640, slots_resident=600, hit_frac=0.8)
    return mx


def test_publication_reads_as_live_and_leaves_no_temporary(tmp_path):
    """monitor.rs:42-58."""
    path = tmp_path / "metrics.json"
    mx = demo(path)
    mx.publish()
    kind, s = moert.read_metrics(path)
    assert kind == "live"
    assert s["schema"] == moert.METRICS_SCHEMA and s["pid"] == os.getpid()
    assert s["state"] == {"kind": "generating", "tokens": 120, "max_tokens": 400}
    assert s["cache"]["slots_total"] == 640 and s["cache"]["hit_frac"] == 0.8
    assert os.listdir(tmp_path) == ["metrics.json"]
    mx.close()


def test_old_publication_reads_as_stopped_runtime(tmp_path):
    """monitor.rs:60-69."""
    path = tmp_path / "metrics.json"
    demo(path).publish()
    kind, s = moert.read_metrics(path, moert.metrics_now_ms() + moert.METRICS_STALE_MS + 1000)
    assert kind == "stale" and s["model"]["name"] == "teste"


def test_absent_invalid_or_other_schema(tmp_path):
    """monitor.rs:71-83."""
    path = tmp_path / "metrics.json"
    assert moert.read_metrics(path) == ("absent", None)
    path.write_bytes(b"{meio json")
    assert moert.read_metrics(path)[0] == "invalid"
    mx = demo(path)
    mx.publish()
    s = json.loads(path.read_text())
    s["schema"] = moert.METRICS_SCHEMA + 1
    path.write_text(json.dumps(s))
    kind, msg = moert.read_metrics(path)
    assert kind == "invalid" and "schema" in msg


def test_snapshot_has_the_reference_layout_in_field_order(tmp_path):
    """Every field of Snapshot and its sections in declaration order (snapshot.rs:18-139), ts_ms and pid set at
    publication, started_ms at creation."""
    t0 = moert.metrics_now_ms()
    mx = demo(tmp_path / "m.json")
    s = json.loads(mx.json())
    assert list(s) == SNAPSHOT_KEYS
    for sec, keys in SECTION_KEYS.items():
        assert list(s[sec]) == keys, sec
    assert t0 - 5 <= s["started_ms"] <= s["ts_ms"] <= moert.metrics_now_ms() + 5
    assert s["requests"] == [] and s["settings"] == {} and s["events"] == []
    # integral f64 values carry a fraction, as serde_json writes them
    assert '"decode_now":0.0' in mx.json()


@pytest.mark.parametrize("kind,a,b,msg,want", [
    (moert.STATE_IDLE, 0, 0, None, {"kind": "idle"}),
    (moert.STATE_READING, 3, 10, None, {"kind": "reading", "done": 3, "total": 10}),
    (moert.STATE_GENERATING, 5, 64, None, {"kind": "generating", "tokens": 5, "max_tokens": 64}),
    (moert.STATE_QUEUED, 2, 0, None, {"kind": "queued", "waiting": 2}),
    (moert.STATE_ERROR, 0, 0, "logits divergem", {"kind": "error", "message": "logits divergem"}),
])
def test_state_is_tagged_by_kind(tmp_path, kind, a, b, msg, want):
    """State as serde's internally tagged enum, snake_case (snapshot.rs:60-72)."""
    mx = moert.Metrics(tmp_path / "m.json")
    mx.set_state(kind, a, b, msg)
    assert json.loads(mx.json())["state"] == want


def test_requests_newest_first_events_oldest_first_and_both_bounded(tmp_path):
    mx = moert.Metrics(tmp_path / "m.json")
    for i in range(40):
        mx.add_request(status="ok" if i % 2 else "erro", started_ms=i, prompt_tokens=10 + i, output_tokens=i,
                       duration_ms=7, prefill_tok_s=1.5, decode_tok_s=float(i))
    for i in range(70):
        mx.event("info", f"e{i}")
    s = json.loads(mx.json())
    assert [r["started_ms"] for r in s["requests"]] == list(range(39, 7, -1))
    assert s["requests"][0] == {"started_ms": 39, "prompt_tokens": 49, "reused_tokens": 0, "output_tokens": 39,
                                "duration_ms": 7, "prefill_tok_s": 1.5, "decode_tok_s": 39.0, "status": "ok"}
    assert [e["message"] for e in s["events"]] == [f"e{i}" for i in range(6, 70)]
    assert all(e["level"] == "info" and e["ts_ms"] > 0 for e in s["events"])


def test_settings_are_a_sorted_map_and_later_values_replace_earlier(tmp_path):
    mx = moert.Metrics(tmp_path / "m.json")
    for k, v in [("threads", "16"), ("política", "lru"), ("b", "1"), ("a", "x"), ("b", "2")]:
        mx.setting(k, v)
    raw = mx.json()
    s = json.loads(raw)
    assert list(s["settings"].items()) == [("a", "x"), ("b", "2"), ("política", "lru"), ("threads", "16")]


def test_strings_are_escaped_and_invalid_utf8_is_replaced(tmp_path):
    """Quotes, backslashes, control characters and non-ASCII text survive a JSON round trip; bytes that are not
    UTF-8 become U+FFFD (a Rust String cannot hold them)."""
    mx = moert.Metrics(tmp_path / "m.json")
    text = 'aspas " barra \\ nova\nlinha\ttab \x01 ç 漢 🙂'
    mx.set_model(text, 1, 2, 3)
    assert json.loads(mx.json())["model"]["name"] == text
    moert.check(moert.lib().moert_metrics_event(mx.h, b"erro", b"ok \xff\xfe fim \xe2\x82"))
    moert.check(moert.lib().moert_metrics_setting(mx.h, b"k\xc0\xaf", b"\xed\xa0\x80"))  # overlong, surrogate
    s = json.loads(mx.json())
    assert s["events"][0]["message"] == "ok �� fim ��"
    assert s["settings"] == {"k��": "���"}


def test_non_finite_floats_are_null_and_values_round_trip(tmp_path):
    mx = moert.Metrics(tmp_path / "m.json")
    vals = dict(decode_now=1 / 3, decode_last=float("nan"), prefill_now=float("inf"), prefill_request=1e-300)
    mx.set_speed(**vals)
    sp = json.loads(mx.json())["speed"]
    assert sp["decode_now"] == 1 / 3 and sp["prefill_request"] == 1e-300
    assert sp["decode_last"] is None and sp["prefill_now"] is None
    mx.set_window(exposure_frac=0.125, gpu_wait_frac=math.pi, ms_per_token=2.0)
    assert json.loads(mx.json())["window"] == {"exposure_frac": 0.125, "gpu_wait_frac": math.pi, "ms_per_token": 2.0}


def test_default_path_follows_xdg_runtime_dir(tmp_path, monkeypatch):
    """default_path (snapshot.rs:146-156); the directory is created."""
    monkeypatch.setenv("XDG_RUNTIME_DIR", str(tmp_path / "run"))
    mx = moert.Metrics()
    assert mx.path == str(tmp_path / "run" / "moe-rt" / "metrics.json")
    mx.publish()
    assert moert.read_metrics(mx.path)[0] == "live"
    monkeypatch.setenv("XDG_RUNTIME_DIR", "")
    assert moert.Metrics().path == f"/tmp/moe-rt-{os.stat('/proc/self').st_uid}/metrics.json"


def test_failures_are_errors_and_keep_the_previous_file(tmp_path):
    blocker = tmp_path / "file"
    blocker.write_text("x")
    with pytest.raises(moert.MoertError, match="directory"):
        moert.Metrics(blocker / "metrics.json")
    path = tmp_path / "d" / "metrics.json"
    mx = demo(path)
    mx.publish()
    before = path.read_bytes()
    (tmp_path / "d" / "metrics.json.tmp-x").mkdir()  # an unrelated entry: the directory cannot be removed
    os.rename(tmp_path / "d", tmp_path / "gone")
    with pytest.raises(moert.MoertError, match="cannot create"):
        mx.publish()
    assert (tmp_path / "gone" / "metrics.json").read_bytes() == before


def test_a_concurrent_reader_never_sees_half_a_file(tmp_path):
    """The point of the temporary file + rename: a reader polling while snapshots are published sees either no file
    or a whole snapshot."""
    path = tmp_path / "metrics.json"
    mx = demo(path)
    for i in range(64):
        mx.setting(f"key {i}", "v" * 200)
    stop = threading.Event()
    seen = {"live": 0, "absent": 0, "other": []}

    def reader():
        while not stop.is_set():
            kind, s = moert.read_metrics(path)
            if kind in ("live", "absent"):
                seen[kind] += 1
            else:
                seen["other"].append((kind, s))

    t = threading.Thread(target=reader)
    t.start()
    for i in range(300):
        mx.set_state(moert.STATE_GENERATING, i, 300)
        mx.publish()
    stop.set()
    t.join()
    assert seen["other"] == [] and seen["live"] > 0
    assert moert.read_metrics(path)[1]["state"]["tokens"] == 299
