"""The C ABI library loads and exports every entry point include/moert.h declares; host-side logic (quantisers,
synthetic data, config parsing, argument refusal) works without a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

import moert

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "moert.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moert_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    names = header_functions()
    assert len(names) >= 30
    raw = ctypes.CDLL(moert.LIB_PATH)
    missing = [n for n in names if not hasattr(raw, n)]
    assert not missing, missing
    assert sorted(moert.EXPORTED) == names  # the Python binding covers exactly the header


def test_device_info_works_without_a_device():
    n, name = moert.device_info()
    assert n >= 0 and isinstance(name, str)


@pytest.mark.parametrize("dtype,levels,steps", [(moert.Q8_0, 127, 0.5), (moert.Q4_0, 8, 1.0)])
def test_quantiser_round_trip_error_is_bounded_by_the_step(dtype, levels, steps):
    """Q8_0: half a step. Q4_0 codes span [-8, 7] d with d = max / -8, so a value of the opposite sign and the same
    magnitude as the block maximum clamps at code 15: one step."""
    import oracle
    x = moert.synth_normal(5, 0, 32 * 4096, 0.02)
    blob = moert.quantize(x, dtype)
    assert blob.size == moert.dtype_bytes(dtype, x.size)
    y = oracle.dequant(blob, dtype, x.size).reshape(-1, 32)
    xb = x.reshape(-1, 32).astype(np.float64)
    amax = np.abs(xb).max(axis=1, keepdims=True)
    step = amax / levels
    assert np.all(np.abs(y - xb) <= step * steps + amax * 2e-3 + 1e-12)


def test_synthetic_data_is_deterministic_and_range_independent():
    a = moert.synth_normal(9, 3, 100_003)
    b = moert.synth_normal(9, 3, 100_003)
    assert np.array_equal(a, b)
    c = moert.synth_normal(9, 4, 1000)
    assert not np.array_equal(a[:1000], c)
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1.0) < 0.02
    q1 = moert.synth_quantized(9, 3, 1 << 20, 0.02, moert.Q8_0)
    q2 = moert.synth_quantized(9, 3, 1 << 20, 0.02, moert.Q8_0)
    assert np.array_equal(q1, q2)


def test_config_from_json_reads_granite_and_refuses_unsupported_variants():
    """tests/model.rs:12-24."""
    base = {"model_type": "granitemoe", "hidden_size": 256, "intermediate_size": 128, "num_hidden_layers": 2,
            "num_attention_heads": 4, "num_key_value_heads": 2, "vocab_size": 33, "num_local_experts": 4,
            "num_experts_per_tok": 2, "rope_theta": 10000.0, "rms_norm_eps": 1e-6, "embedding_multiplier": 2.0,
            "residual_multiplier": 0.5, "attention_multiplier": 0.125, "logits_scaling": 4.0, "rope_scaling": None,
            "attention_bias": False, "tie_word_embeddings": True}
    c = moert.Config.from_json(base)
    assert (c.hidden, c.heads, c.kv_heads, c.head_dim, c.vocab) == (256, 4, 2, 64, 33)
    for key, val in [("model_type", "llama"), ("rope_scaling", {"type": "linear", "factor": 2.0}),
                     ("attention_bias", True), ("tie_word_embeddings", False)]:
        with pytest.raises(ValueError):
            moert.Config.from_json({**base, key: val})


def test_model_create_refuses_unsupported_shapes_before_touching_the_device():
    m = moert.SynthModel(moert.Config(**moert.TINY))
    for bad in [dict(head_dim=128), dict(max_len=100), dict(top_k=9)]:
        cfg = moert.Config(**{**moert.TINY, **{k: v for k, v in bad.items() if k != "max_len"}})
        h = ctypes.c_void_p()
        rc = moert.lib().moert_model_create(ctypes.byref(cfg.c()), ctypes.byref(m.weights()),
                                            bad.get("max_len", 128), 8, ctypes.byref(h))
        assert rc == -2, bad
        assert moert.lib().moert_last_error()


def test_step_bytes_matches_the_published_roofline_figures():
    """Algorithmic bytes per decode step of the long-context 3B workload: 938,341,152 + 65,536 n with a Q8_0 head,
    and 603,451,392 + 49,152 n for the 1B model with an fp32 head."""
    c3 = moert.Config(**moert.GRANITE_3B)
    assert moert.step_bytes(c3, moert.Q8_0, moert.Q8_0, 0) == 938_341_152
    assert moert.step_bytes(c3, moert.Q8_0, moert.Q8_0, 1) - moert.step_bytes(c3, moert.Q8_0, moert.Q8_0, 0) == 65_536
    c1 = moert.Config(**moert.GRANITE_1B)
    assert moert.step_bytes(c1, moert.Q8_0, moert.F32, 0) == 603_451_392
    assert moert.step_bytes(c1, moert.Q8_0, moert.F32, 1) - moert.step_bytes(c1, moert.Q8_0, moert.F32, 0) == 49_152
