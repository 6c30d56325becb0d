"""Checkpoint loading through the C ABI (host only): the safetensors reader (the reference's cases,
rust/moe-rt/tests/block.rs:132-180), config.json (model.rs:34-61, tests/model.rs:12-24) and the Granite host model with
quantize-on-load (HostModel::load, model.rs:100-132), checked tensor by tensor against BF16 rounding + the quantiser."""
import ctypes
import json
import os

import numpy as np
import pytest

import moert

TINY_JSON = {
    "model_type": "granitemoe", "hidden_size": 256, "intermediate_size": 128, "num_hidden_layers": 2,
    "num_attention_heads": 4, "num_key_value_heads": 2, "vocab_size": 33, "num_local_experts": 4,
    "num_experts_per_tok": 2, "rope_theta": 10000.0, "rms_norm_eps": 1e-6, "embedding_multiplier": 2.0,
    "residual_multiplier": 0.5, "attention_multiplier": 0.125, "logits_scaling": 4.0, "rope_scaling": None,
    "attention_bias": False, "tie_word_embeddings": True}


def values(n, seed):
    """The reference's xorshift test values in [-1, 1) (tests/common/mod.rs:28-38)."""
    out = np.empty(n, np.float32)
    s = (seed | 1) & 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        out[i] = np.float32((s >> 40) / float(1 << 23)) * np.float32(2.0) - np.float32(1.0)
    return out


def widen(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def test_reader_reads_bf16_and_refuses_other_dtypes_missing_tensors_and_bad_offsets(tmp_path):
    """tests/block.rs:132-150."""
    v = moert.bf16_bits(values(6, 3))
    path = tmp_path / "model.safetensors"
    moert.write_safetensors(path, [("a", "BF16", [2, 3], v.tobytes()), ("b", "F32", [1], bytes(4))])
    ck = moert.Checkpoint(tmp_path)
    assert ck.tensor("a") == ("BF16", (2, 3))
    assert np.array_equal(ck.bf16("a"), v.reshape(2, 3))
    with pytest.raises(moert.MoertError, match="F32"):
        ck.bf16("b")
    with pytest.raises(moert.MoertError, match="missing"):
        ck.bf16("c")
    ck.close()
    raw = path.read_bytes()
    path.write_bytes(raw[:-6])  # offsets past the end of the file
    with pytest.raises(moert.MoertError, match="ends past the data section"):
        moert.Checkpoint(tmp_path)


@pytest.mark.parametrize("entry", [
    {"dtype": "BF16", "shape": [2], "data_offsets": [0]},
    {"dtype": "BF16", "shape": [2], "data_offsets": []},
    {"dtype": "BF16", "shape": [2], "data_offsets": [0, 4, 8]},
    {"dtype": "BF16", "shape": [2], "data_offsets": ["0", 4]},
    {"dtype": "BF16", "shape": [2], "data_offsets": [2 ** 64 - 1, 2 ** 64 - 1]},
    {"dtype": "BF16", "shape": [2], "data_offsets": [2 ** 64 - 5, 2 ** 64 - 1]},
    {"dtype": "BF16", "shape": [-2], "data_offsets": [0, 4]},
    {"shape": [2], "data_offsets": [0, 4]},
    {"dtype": "BF16", "data_offsets": [0, 4]},
    {"dtype": "BF16", "shape": [2], "data_offsets": [4, 0]},
])
def test_reader_refuses_malformed_headers(tmp_path, entry):
    """tests/block.rs:152-175: every malformed entry is an error, never a crash."""
    head = json.dumps({"a": entry}).encode()
    (tmp_path / "model.safetensors").write_bytes(len(head).to_bytes(8, "little") + head + bytes(16))
    with pytest.raises(moert.MoertError):
        moert.Checkpoint(tmp_path)


def test_reader_refuses_an_overflowing_shape_on_read_and_broken_files_on_open(tmp_path):
    """A shape whose byte count overflows is an error when read (tests/block.rs:176-179); so are a header that is
    not JSON, a header length beyond 100 MiB and a directory without safetensors files."""
    head = json.dumps({"a": {"dtype": "BF16", "shape": [2 ** 64 - 1, 4], "data_offsets": [0, 4]}}).encode()
    p = tmp_path / "model.safetensors"
    p.write_bytes(len(head).to_bytes(8, "little") + head + bytes(16))
    ck = moert.Checkpoint(tmp_path)
    buf = np.zeros(2, np.uint16)
    with pytest.raises(moert.MoertError, match="byte count differs"):
        moert.check(moert.lib().moert_checkpoint_read_bf16(ck.h, b"a", moert.ptr(buf), 2))
    ck.close()
    for raw in (b"\x05\x00\x00\x00\x00\x00\x00\x00{abc}", (200 << 20).to_bytes(8, "little") + b"{}", b"\x01\x00"):
        p.write_bytes(raw)
        with pytest.raises(moert.MoertError):
            moert.Checkpoint(tmp_path)
    p.unlink()
    with pytest.raises(moert.MoertError, match="no \\*.safetensors"):
        moert.Checkpoint(tmp_path)


def test_config_from_json_equals_the_python_statement_and_refuses_unsupported_variants():
    """Config::from_json (model.rs:34-61); refusals as tests/model.rs:12-24."""
    c = moert.config_from_json_native(json.dumps(TINY_JSON))
    p = moert.Config.from_json(TINY_JSON)
    assert bytes(c.c()) == bytes(p.c())
    assert c.head_dim == 64
    for change in ({"model_type": "llama"}, {"rope_scaling": {"type": "linear"}}, {"attention_bias": True},
                   {"tie_word_embeddings": False}):
        with pytest.raises(moert.MoertError):
            moert.config_from_json_native(json.dumps({**TINY_JSON, **change}))
    missing = dict(TINY_JSON)
    del missing["vocab_size"]
    with pytest.raises(moert.MoertError, match="vocab_size"):
        moert.config_from_json_native(json.dumps(missing))
    with pytest.raises(moert.MoertError):
        moert.config_from_json_native('{"model_type": "granitemoe",')
    assert moert.config_from_json_native(json.dumps({**TINY_JSON, "head_dim": 32})).head_dim == 32


def granite_checkpoint(path, cfg, seed=10, files=2):
    """A synthetic Granite-MoE checkpoint in BF16 (tests/common/mod.rs:79-131, values N(0, 0.05) from the engine's
    seeded generator, norm weights 1 + N(0, 0.05)), split over `files` safetensors files. Returns {name: bits}."""
    h, i, e, d = cfg.hidden, cfg.inter, cfg.experts, cfg.head_dim
    qd, kvd = cfg.heads * d, cfg.kv_heads * d
    shapes = [("model.embed_tokens.weight", [cfg.vocab, h]), ("model.norm.weight", [h])]
    for l in range(cfg.layers):
        p = f"model.layers.{l}"
        shapes += [(f"{p}.input_layernorm.weight", [h]), (f"{p}.post_attention_layernorm.weight", [h]),
                   (f"{p}.self_attn.q_proj.weight", [qd, h]), (f"{p}.self_attn.k_proj.weight", [kvd, h]),
                   (f"{p}.self_attn.v_proj.weight", [kvd, h]), (f"{p}.self_attn.o_proj.weight", [h, qd]),
                   (f"{p}.block_sparse_moe.router.layer.weight", [e, h]),
                   (f"{p}.block_sparse_moe.input_linear.weight", [e, 2 * i, h]),
                   (f"{p}.block_sparse_moe.output_linear.weight", [e, h, i])]
    bits = {}
    for k, (name, shape) in enumerate(shapes):
        n = int(np.prod(shape))
        norm = len(shape) == 1
        v = moert.synth_normal(seed, k, n, 0.05, 1.0 if norm else 0.0)
        bits[name] = moert.bf16_bits(v).reshape(shape)
    per = (len(shapes) + files - 1) // files
    for f in range(files):
        chunk = shapes[f * per:(f + 1) * per]
        moert.write_safetensors(os.path.join(path, f"model-{f + 1:05d}-of-{files:05d}.safetensors"),
                                [(n, "BF16", s, bits[n].tobytes()) for n, s in chunk])
    return bits


def _blob(t, nbytes):
    return np.frombuffer(ctypes.string_at(t.data, nbytes), np.uint8)


@pytest.mark.parametrize("wdtype,edtype", [(moert.Q8_0, moert.Q8_0), (moert.Q4_0, moert.F32), (moert.F32, moert.Q4_0)])
def test_loaded_model_is_the_bf16_checkpoint_quantised_on_load(tmp_path, wdtype, edtype):
    """HostModel::load over a two-file checkpoint: every matrix equals its BF16 values widened to f32 and quantised
    to the requested dtype (byte for byte), every norm weight its BF16 value widened."""
    cfg = moert.Config(**{k: v for k, v in moert.TINY.items()})
    bits = granite_checkpoint(str(tmp_path), cfg)
    ck = moert.Checkpoint(tmp_path)
    m = moert.LoadedModel(ck, cfg, wdtype, edtype)
    w = m.weights()
    emb = moert.quantize(widen(bits["model.embed_tokens.weight"]).ravel(), edtype)
    assert w.embed.dtype == edtype and np.array_equal(_blob(w.embed, emb.nbytes), emb.view(np.uint8))
    norm = np.ctypeslib.as_array(ctypes.cast(w.norm, ctypes.POINTER(ctypes.c_float)), (cfg.hidden,))
    assert np.array_equal(norm, widen(bits["model.norm.weight"]))
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
             "router": "block_sparse_moe.router.layer", "gate_up": "block_sparse_moe.input_linear",
             "down": "block_sparse_moe.output_linear"}
    for l in range(cfg.layers):
        L = w.layers[l]
        for field, name in names.items():
            want = moert.quantize(widen(bits[f"model.layers.{l}.{name}.weight"]).ravel(), wdtype)
            t = getattr(L, field)
            assert t.dtype == wdtype
            assert np.array_equal(_blob(t, want.nbytes), want.view(np.uint8)), (l, field)
        for field, name in (("ln_attn", "input_layernorm"), ("ln_moe", "post_attention_layernorm")):
            got = np.ctypeslib.as_array(ctypes.cast(getattr(L, field), ctypes.POINTER(ctypes.c_float)), (cfg.hidden,))
            assert np.array_equal(got, widen(bits[f"model.layers.{l}.{name}.weight"]))
        assert not L.router_bias
    m.close()
    ck.close()


def test_loader_refuses_wrong_shapes_and_missing_tensors(tmp_path):
    """A shape that differs from config.json names the tensor (model.rs:102-108); a missing tensor is refused."""
    cfg = moert.Config(**moert.TINY)
    bits = granite_checkpoint(str(tmp_path), cfg, files=1)
    ck = moert.Checkpoint(tmp_path)
    wrong = moert.Config(**{**moert.TINY, "inter": 64})
    with pytest.raises(moert.MoertError, match="input_linear"):
        moert.LoadedModel(ck, wrong, moert.Q8_0, moert.Q8_0)
    more = moert.Config(**{**moert.TINY, "layers": 3})
    with pytest.raises(moert.MoertError, match="model.layers.2"):
        moert.LoadedModel(ck, more, moert.Q8_0, moert.Q8_0)
    ck.close()
    assert len(bits) == 2 + 9 * cfg.layers
