"""Python binding of libmoert (include/moert.h), the gfx950 Granite-MoE decode engine.

Mirrors the host API of the reference crate rust/moe-rt (brenoperucchi/lastro-rust):
  Config            <- model.rs:14-61 (Config / from_json)
  SynthModel        <- model.rs:87-132 (HostModel) built from seeded synthetic weights instead of a checkpoint
  GpuModel          <- gpu_model.rs:180-445 (upload, step, reset) + cuda_backend.rs model mode (read_kv, reset)
  GpuBlock          <- gpu.rs:368-541 (GpuLayer) / block.rs:56-62 (forward_cpu)
  router_topk       <- route.rs:18-75 / block.rs:81-89
  argmax            <- bin/m1b-gulosa.rs:22-24
The library is required: every entry point raises if libmoert.so is missing or a call fails.
"""
from __future__ import annotations

import ctypes
import json
import math
import os
import time
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

F32, Q8_0, Q4_0 = 0, 1, 2
DTYPE_NAMES = {F32: "f32", Q8_0: "q8_0", Q4_0: "q4_0"}

(K_EMBED, K_QKV, K_ATTN_SPLIT, K_ATTN_COMBINE, K_OPROJ, K_ROUTE_UP, K_EXPERT_DOWN, K_HEAD,
 K_HEAD_ARGMAX, K_ATTN_BLOCK, K_MOE_XCD, K_MOE_COMBINE, K_LAYER, K_LAYER_COMBINE) = range(14)
KERNEL_NAMES = ["embed", "qkv", "attn_split", "attn_combine", "oproj", "route_up", "expert_down", "head",
                "head_argmax", "attn_block", "moe_xcd", "moe_combine", "layer",
                "layer_combine"]   # kernel classes of a decode step (the same for a cached model)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmoert.so")
TIMELINE_LIB_PATH = os.path.join(_HERE, "libmoert_tl.so")  # measurement build (phase timeline), see timeline.py
TL_WORDS = 12  # words of a workgroup's timeline record: start, latest start, 9 phase ends, latest end

E_NAMES = {-1: "DEVICE", -2: "CONFIG", -3: "POISONED", -4: "FULL", -5: "RANGE"}
E_DEVICE, E_CONFIG, E_POISONED, E_FULL, E_RANGE = -1, -2, -3, -4, -5


class MoertError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"moert error {code} ({E_NAMES.get(code, '?')}): {msg}")
        self.code = code


class moert_config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("hidden", "inter", "layers", "heads", "kv_heads", "head_dim", "vocab", "experts", "top_k")] + \
               [(n, ctypes.c_float) for n in
                ("rope_theta", "eps", "embedding_multiplier", "residual_multiplier", "attention_multiplier",
                 "logits_scaling")]


class moert_tensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int)]


class moert_layer_weights(ctypes.Structure):
    _fields_ = [("ln_attn", ctypes.c_void_p), ("ln_moe", ctypes.c_void_p), ("q", moert_tensor),
                ("k", moert_tensor), ("v", moert_tensor), ("o", moert_tensor), ("router", moert_tensor),
                ("router_bias", ctypes.c_void_p), ("gate_up", moert_tensor), ("down", moert_tensor)]


class moert_cache_counters(ctypes.Structure):
    _fields_ = [(n, ctypes.c_ulonglong) for n in
                ("needed", "hits", "copies", "prefetched", "cpu", "dropped", "deferred", "bytes_copied")] + \
               [("slots", ctypes.c_int)]


class moert_metrics_speed(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in ("decode_now", "decode_last", "prefill_now", "prefill_request")]


class moert_metrics_cache(ctypes.Structure):
    _fields_ = [("slots_total", ctypes.c_uint32), ("slots_resident", ctypes.c_uint32),
                ("slots_loading", ctypes.c_uint32), ("hit_frac", ctypes.c_double), ("copy_frac", ctypes.c_double),
                ("cpu_frac", ctypes.c_double), ("copies_inflight", ctypes.c_uint32), ("h2d_gbs", ctypes.c_double),
                ("total_hits", ctypes.c_uint64), ("total_copies", ctypes.c_uint64), ("total_cpu", ctypes.c_uint64)]


class moert_metrics_window(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in ("exposure_frac", "gpu_wait_frac", "ms_per_token")]


class moert_metrics_request(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in
                ("started_ms", "prompt_tokens", "reused_tokens", "output_tokens", "duration_ms")] + \
               [("prefill_tok_s", ctypes.c_double), ("decode_tok_s", ctypes.c_double), ("status", ctypes.c_char_p)]


class moert_model_weights(ctypes.Structure):
    _fields_ = [("embed", moert_tensor), ("norm", ctypes.c_void_p),
                ("layers", ctypes.POINTER(moert_layer_weights))]


_lib = None


def lib() -> ctypes.CDLL:
    """Loads libmoert.so (built by `make -C lastro-rust_amd`); raises if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is missing: build it with `make -C {_HERE}`")
        L = ctypes.CDLL(LIB_PATH)
        vp, ip, fp, i, f, sz = ctypes.c_void_p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_float), \
            ctypes.c_int, ctypes.c_float, ctypes.c_size_t
        u64 = ctypes.c_uint64
        sig = {
            "moert_last_error": (ctypes.c_char_p, []),
            "moert_device_info": (i, [ip, ctypes.c_char_p, i]),
            "moert_model_create": (i, [ctypes.POINTER(moert_config), ctypes.POINTER(moert_model_weights), i, i,
                                       ctypes.POINTER(vp)]),
            "moert_model_destroy": (i, [vp]),
            "moert_model_create_cached": (i, [ctypes.POINTER(moert_config), ctypes.POINTER(moert_model_weights), i,
                                              i, i, ctypes.POINTER(vp)]),
            "moert_cache_stats": (i, [vp, ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(ctypes.c_ulonglong)]),
            "moert_cache_clear": (i, [vp]),
            "moert_cache_fill": (i, [vp, ctypes.POINTER(ctypes.c_int)]),
            "moert_cache_prefetch": (i, [vp, i, vp, i, ctypes.POINTER(ctypes.c_int)]),
            "moert_cache_prefetch_mode": (i, [vp, i]),
            "moert_cache_predictions": (i, [vp, i, i, vp]),
            "moert_cache_token_counts": (i, [vp, i, i, vp]),
            "moert_batched_mode": (i, [vp, i]),
            "moert_model_create_hybrid": (i, [ctypes.POINTER(moert_config), ctypes.POINTER(moert_model_weights), i,
                                              i, i, i, i, ctypes.POINTER(vp)]),
            "moert_cache_counters_get": (i, [vp, ctypes.POINTER(moert_cache_counters)]),
            "moert_decode_step": (i, [vp, i, vp, vp, vp, ip]),
            "moert_generate": (i, [vp, vp, i, i, vp, vp]),
            "moert_step_batched": (i, [vp, vp, i, vp, ip]),
            "moert_prefill": (i, [vp, vp, i, vp, ip]),
            "moert_reset_sequence": (i, [vp]),
            "moert_kv_prefill_fp16": (i, [vp, i, vp, vp, i]),
            "moert_set_position": (i, [vp, i]),
            "moert_get_position": (i, [vp, ip]),
            "moert_read_kv_fp16": (i, [vp, i, vp, vp, i]),
            "moert_read_hidden": (i, [vp, vp]),
            "moert_read_logits": (i, [vp, vp]),
            "moert_time_steps": (i, [vp, i, i, ctypes.POINTER(ctypes.c_double)]),
            "moert_time_kernel": (i, [vp, i, i, ctypes.POINTER(ctypes.c_double), ip]),
            "moert_fault_inject": (i, [vp, ctypes.c_uint]),
            "moert_model_path": (i, [vp, ip, ip, ip]),
            "moert_timeline_step": (i, [vp, vp, vp, vp, i, ip]),
            "moert_block_create": (i, [i, i, i, i, ctypes.POINTER(moert_tensor), vp, ctypes.POINTER(moert_tensor),
                                       ctypes.POINTER(moert_tensor), ctypes.POINTER(vp)]),
            "moert_block_destroy": (i, [vp]),
            "moert_block_forward": (i, [vp, vp, vp, vp, vp]),
            "moert_block_time": (i, [vp, i, ctypes.POINTER(ctypes.c_double)]),
            "moert_block_forward_batched": (i, [vp, i, vp, vp, vp, vp]),
            "moert_block_experts_in_step": (i, [vp, ip]),
            "moert_block_batched_kernel": (i, [vp, i]),
            "moert_block_fault_inject": (i, [vp, ctypes.c_uint]),
            "moert_block_time_batched": (i, [vp, i, i, i, vp]),
            "moert_router_topk": (i, [vp, i, i, vp, vp]),
            "moert_argmax": (i, [vp, i, ip]),
            "moert_gemv": (i, [ctypes.POINTER(moert_tensor), i, i, vp, vp]),
            "moert_dequant": (i, [ctypes.POINTER(moert_tensor), i, i, vp]),
            "moert_rmsnorm": (i, [vp, vp, i, f, vp]),
            "moert_rope": (i, [vp, i, i, f, i]),
            "moert_attn_decode": (i, [vp, vp, vp, i, i, i, i, i, f, i, vp]),
            "moert_attn_decode_noalloc": (i, [vp, vp, vp, i, i, i, i, i, f, i, vp, vp]),
            "moert_exp_device": (i, [vp, vp, i]),
            "moert_copy_probe": (i, [sz, i, ctypes.POINTER(ctypes.c_double)]),
            "moert_read_probe": (i, [sz, i, ctypes.POINTER(ctypes.c_double)]),
            "moert_h2d_probe": (i, [sz, i, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
            "moert_quantize": (i, [vp, sz, i, vp]),
            "moert_dtype_bytes": (sz, [i, sz]),
            "moert_synth_normal": (i, [u64, u64, sz, f, f, vp]),
            "moert_synth_quantized": (i, [u64, u64, sz, f, i, vp]),
            "moert_synth_fp16": (i, [u64, u64, sz, f, vp]),
            "moert_config_from_json": (i, [ctypes.c_char_p, sz, ctypes.POINTER(moert_config)]),
            "moert_checkpoint_open": (i, [ctypes.c_char_p, ctypes.POINTER(vp)]),
            "moert_checkpoint_close": (i, [vp]),
            "moert_checkpoint_tensor": (i, [vp, ctypes.c_char_p, ctypes.c_char_p, i, vp, i, ip]),
            "moert_checkpoint_read_bf16": (i, [vp, ctypes.c_char_p, vp, sz]),
            "moert_checkpoint_load": (i, [vp, ctypes.POINTER(moert_config), i, i, ctypes.POINTER(vp)]),
            "moert_host_model_weights": (ctypes.POINTER(moert_model_weights), [vp]),
            "moert_host_model_config": (i, [vp, ctypes.POINTER(moert_config)]),
            "moert_host_model_destroy": (i, [vp]),
            "moert_metrics_create": (i, [ctypes.c_char_p, ctypes.POINTER(vp)]),
            "moert_metrics_destroy": (i, [vp]),
            "moert_metrics_path": (i, [vp, ctypes.c_char_p, i]),
            "moert_metrics_set_model": (i, [vp, ctypes.c_char_p, i, i, i]),
            "moert_metrics_set_state": (i, [vp, i, u64, u64, ctypes.c_char_p]),
            "moert_metrics_set_speed": (i, [vp, ctypes.POINTER(moert_metrics_speed)]),
            "moert_metrics_set_context": (i, [vp, u64, u64]),
            "moert_metrics_set_cache": (i, [vp, ctypes.POINTER(moert_metrics_cache)]),
            "moert_metrics_set_window": (i, [vp, ctypes.POINTER(moert_metrics_window)]),
            "moert_metrics_add_request": (i, [vp, ctypes.POINTER(moert_metrics_request)]),
            "moert_metrics_setting": (i, [vp, ctypes.c_char_p, ctypes.c_char_p]),
            "moert_metrics_event": (i, [vp, ctypes.c_char_p, ctypes.c_char_p]),
            "moert_metrics_json": (i, [vp, ctypes.c_char_p, sz, ctypes.POINTER(sz)]),
            "moert_metrics_publish": (i, [vp]),
            "moert_model_attach_metrics": (i, [vp, vp, i]),
            "moert_placement_create": (i, [i, i, i, i, i, ctypes.POINTER(vp)]),
            "moert_placement_destroy": (i, [vp]),
            "moert_placement_step": (i, [vp, vp, i, ip, ip]),
            "moert_placement_counters": (i, [vp, ctypes.POINTER(moert_cache_counters)]),
            "moert_placement_table": (i, [vp, vp]),
            "moert_freq_create": (i, [i, i, ctypes.POINTER(vp)]),
            "moert_freq_destroy": (i, [vp]),
            "moert_freq_touch": (i, [vp, i, u64]),
            "moert_freq_score": (i, [vp, i, ctypes.POINTER(ctypes.c_double)]),
            "moert_freq_clear": (i, [vp]),
            "moert_tokenizer_load": (i, [ctypes.c_char_p, ctypes.POINTER(vp)]),
            "moert_tokenizer_from_json": (i, [ctypes.c_char_p, sz, ctypes.POINTER(vp)]),
            "moert_tokenizer_destroy": (i, [vp]),
            "moert_tokenizer_vocab_size": (i, [vp, ip]),
            "moert_tokenizer_encode": (i, [vp, ctypes.c_char_p, sz, vp, sz, ctypes.POINTER(sz)]),
            "moert_tokenizer_decode": (i, [vp, vp, sz, i, ctypes.c_char_p, sz, ctypes.POINTER(sz)]),
            "moert_tokenizer_pretokenize": (i, [ctypes.c_char_p, sz, vp, sz, ctypes.POINTER(sz)]),
            "moert_chat_render": (i, [ip, ctypes.POINTER(ctypes.c_char_p), i, i, ctypes.c_char_p, ctypes.c_char_p, sz,
                                      ctypes.POINTER(sz)]),
            "moert_format_date": (i, [i, i, i, ctypes.c_char_p, sz]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


EXPORTED = ["moert_last_error", "moert_device_info", "moert_model_create", "moert_model_destroy",
            "moert_model_create_cached", "moert_cache_stats", "moert_cache_clear", "moert_cache_fill",
            "moert_cache_prefetch", "moert_cache_prefetch_mode", "moert_cache_predictions", "moert_cache_token_counts",
            "moert_cache_counters_get", "moert_model_create_hybrid", "moert_batched_mode",
            "moert_decode_step", "moert_generate", "moert_step_batched", "moert_prefill", "moert_reset_sequence",
            "moert_kv_prefill_fp16",
            "moert_set_position", "moert_get_position", "moert_read_kv_fp16", "moert_read_hidden", "moert_read_logits",
            "moert_time_steps", "moert_time_kernel", "moert_fault_inject", "moert_model_path", "moert_timeline_step", "moert_block_create", "moert_block_destroy",
            "moert_block_forward", "moert_block_time", "moert_block_forward_batched",
            "moert_block_experts_in_step", "moert_block_batched_kernel", "moert_block_fault_inject", "moert_block_time_batched", "moert_router_topk", "moert_argmax", "moert_gemv",
            "moert_dequant", "moert_rmsnorm", "moert_rope", "moert_attn_decode", "moert_attn_decode_noalloc",
            "moert_exp_device",
            "moert_copy_probe", "moert_read_probe", "moert_h2d_probe", "moert_quantize", "moert_dtype_bytes", "moert_synth_normal", "moert_synth_quantized",
            "moert_synth_fp16", "moert_config_from_json", "moert_checkpoint_open", "moert_checkpoint_close",
            "moert_checkpoint_tensor", "moert_checkpoint_read_bf16", "moert_checkpoint_load", "moert_host_model_weights",
            "moert_host_model_config", "moert_host_model_destroy", "moert_metrics_create", "moert_metrics_destroy",
            "moert_metrics_path", "moert_metrics_set_model", "moert_metrics_set_state", "moert_metrics_set_speed",
            "moert_metrics_set_context", "moert_metrics_set_cache", "moert_metrics_set_window",
            "moert_metrics_add_request", "moert_metrics_setting", "moert_metrics_event", "moert_metrics_json",
            "moert_metrics_publish", "moert_model_attach_metrics", "moert_placement_create", "moert_placement_destroy",
            "moert_placement_step", "moert_placement_counters", "moert_placement_table", "moert_freq_create",
            "moert_freq_destroy", "moert_freq_touch", "moert_freq_score", "moert_freq_clear", "moert_tokenizer_load",
            "moert_tokenizer_from_json", "moert_tokenizer_destroy", "moert_tokenizer_vocab_size",
            "moert_tokenizer_encode", "moert_tokenizer_decode", "moert_tokenizer_pretokenize", "moert_chat_render",
            "moert_format_date"]


def check(rc: int) -> None:
    if rc != 0:
        raise MoertError(rc, lib().moert_last_error().decode(errors="replace"))


def ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def device_info():
    n = ctypes.c_int(0)
    name = ctypes.create_string_buffer(256)
    check(lib().moert_device_info(ctypes.byref(n), name, 256))
    return n.value, name.value.decode()


def dtype_bytes(dtype: int, n: int) -> int:
    return int(lib().moert_dtype_bytes(dtype, n))


def quantize(x: np.ndarray, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == F32:
        return x.copy()
    out = np.empty(dtype_bytes(dtype, x.size), np.uint8)
    check(lib().moert_quantize(ptr(x), x.size, dtype, ptr(out)))
    return out


def synth_normal(seed: int, stream: int, n: int, scale: float = 1.0, offset: float = 0.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    check(lib().moert_synth_normal(seed, stream, n, scale, offset, ptr(out)))
    return out


def synth_quantized(seed: int, stream: int, n: int, scale: float, dtype: int) -> np.ndarray:
    if dtype == F32:
        return synth_normal(seed, stream, n, scale)
    out = np.empty(dtype_bytes(dtype, n), np.uint8)
    check(lib().moert_synth_quantized(seed, stream, n, scale, dtype, ptr(out)))
    return out


def synth_fp16(seed: int, stream: int, n: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    check(lib().moert_synth_fp16(seed, stream, n, scale, ptr(out)))
    return out


# ----------------------------------------------------------------------------------------------------------------
@dataclass
class Config:
    """Model constants (rust/moe-rt/src/model.rs:14-31)."""
    hidden: int
    inter: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    experts: int
    top_k: int
    rope_theta: float = 10000.0
    eps: float = 1e-6
    embedding_multiplier: float = 12.0
    residual_multiplier: float = 0.22
    attention_multiplier: float = 0.015625
    logits_scaling: float = 6.0

    @staticmethod
    def from_json(v: dict) -> "Config":
        """Config::from_json (model.rs:34-61): refuses non-granitemoe models and unsupported variants."""
        if v.get("model_type") != "granitemoe":
            raise ValueError(f"model_type {v.get('model_type')!r} (expected granitemoe)")
        if v.get("rope_scaling") is not None or v.get("attention_bias") is True or \
                v.get("tie_word_embeddings") is False:
            raise ValueError("unsupported variant (rope_scaling, attention_bias or untied embeddings)")
        h, heads = int(v["hidden_size"]), int(v["num_attention_heads"])
        return Config(hidden=h, inter=int(v["intermediate_size"]), layers=int(v["num_hidden_layers"]), heads=heads,
                      kv_heads=int(v["num_key_value_heads"]), head_dim=int(v.get("head_dim") or h // heads),
                      vocab=int(v["vocab_size"]), experts=int(v["num_local_experts"]),
                      top_k=int(v["num_experts_per_tok"]), rope_theta=float(v["rope_theta"]),
                      eps=float(v["rms_norm_eps"]), embedding_multiplier=float(v["embedding_multiplier"]),
                      residual_multiplier=float(v["residual_multiplier"]),
                      attention_multiplier=float(v["attention_multiplier"]),
                      logits_scaling=float(v["logits_scaling"]))

    def c(self) -> moert_config:
        return moert_config(*[getattr(self, n) for n, _ in moert_config._fields_])

    def inv_freq(self) -> np.ndarray:
        d = np.float32(self.head_dim)
        return np.array([np.float32(1.0) / np.power(np.float32(self.rope_theta), np.float32(2 * j) / d)
                         for j in range(self.head_dim // 2)], np.float32)


# Workload shapes named by the reference's model family (configs of the decode benchmark).
GRANITE_1B = dict(hidden=1024, inter=512, layers=24, heads=16, kv_heads=8, head_dim=64, vocab=49155, experts=32,
                  top_k=8)
GRANITE_3B = dict(hidden=1536, inter=512, layers=32, heads=24, kv_heads=8, head_dim=64, vocab=49155, experts=40,
                  top_k=8)
TINY = dict(hidden=256, inter=128, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=33, experts=4, top_k=2)


@dataclass
class SynthModel:
    """Random-init Granite-MoE weights (HostModel, model.rs:87-132): matrices N(0, std) quantised to `wdtype`,
    norm weights 1 + N(0, std), embedding/head in `embed_dtype`. `zipf_s` adds the router bias
    b_e = -s * ln(rank_e) over a seeded permutation of the experts (skewed expert loads)."""
    cfg: Config
    seed: int = 1234
    wdtype: int = Q8_0
    embed_dtype: int = Q8_0
    std: float = 0.02
    zipf_s: Optional[float] = None
    arrays: dict = field(default_factory=dict)

    def __post_init__(self):
        c, s, a = self.cfg, self.seed, self.arrays
        H, d, I, E = c.hidden, c.head_dim, c.inter, c.experts
        qd, kvd = c.heads * d, c.kv_heads * d
        a["embed"] = synth_quantized(s, 1, c.vocab * H, self.std, self.embed_dtype)
        a["norm"] = synth_normal(s, 2, H, self.std, 1.0)
        for l in range(c.layers):
            b = 100 + 16 * l
            a[f"{l}.ln_attn"] = synth_normal(s, b, H, self.std, 1.0)
            a[f"{l}.ln_moe"] = synth_normal(s, b + 1, H, self.std, 1.0)
            a[f"{l}.q"] = synth_quantized(s, b + 2, qd * H, self.std, self.wdtype)
            a[f"{l}.k"] = synth_quantized(s, b + 3, kvd * H, self.std, self.wdtype)
            a[f"{l}.v"] = synth_quantized(s, b + 4, kvd * H, self.std, self.wdtype)
            a[f"{l}.o"] = synth_quantized(s, b + 5, H * qd, self.std, self.wdtype)
            a[f"{l}.router"] = synth_quantized(s, b + 6, E * H, self.std, self.wdtype)
            a[f"{l}.gate_up"] = synth_quantized(s, b + 7, E * 2 * I * H, self.std, self.wdtype)
            a[f"{l}.down"] = synth_quantized(s, b + 8, E * H * I, self.std, self.wdtype)
            if self.zipf_s is not None:
                a[f"{l}.router_bias"] = zipf_bias(E, s * 1000 + l, self.zipf_s)
        self._struct = None

    def weights(self) -> moert_model_weights:
        """The moert_model_weights struct pointing into the numpy arrays (kept alive by this object)."""
        if self._struct is None:
            c, a = self.cfg, self.arrays
            wd = self.wdtype
            self._layers = (moert_layer_weights * c.layers)()
            for l in range(c.layers):
                L = self._layers[l]
                L.ln_attn = a[f"{l}.ln_attn"].ctypes.data
                L.ln_moe = a[f"{l}.ln_moe"].ctypes.data
                for n in ("q", "k", "v", "o", "router", "gate_up", "down"):
                    setattr(L, n, moert_tensor(a[f"{l}.{n}"].ctypes.data, wd))
                bias = a.get(f"{l}.router_bias")
                L.router_bias = None if bias is None else bias.ctypes.data
            self._struct = moert_model_weights(moert_tensor(a["embed"].ctypes.data, self.embed_dtype),
                                               a["norm"].ctypes.data, self._layers)
        return self._struct

    def weight_bytes(self) -> int:
        return sum(v.nbytes for v in self.arrays.values())


class GpuModel:
    """All weights resident in HBM (GpuModel::upload, gpu_model.rs:191-194) and an fp16 KV cache of max_len; with
    cache_slots, the experts are served from an expert cache of that many HBM slots over a pinned host store
    (GpuModel::upload_cached, gpu_model.rs:197-200)."""

    def __init__(self, model: SynthModel, max_len: int, attn_splits: int = 64, cache_slots: Optional[int] = None,
                 hybrid: Optional[tuple] = None):
        """hybrid = (slots, backlog, cpu_threads): the host-CPU hybrid (moert_model_create_hybrid) instead."""
        self.model, self.cfg, self.max_len = model, model.cfg, max_len
        self.cache_slots = cache_slots
        h = ctypes.c_void_p()
        if hybrid is not None:
            slots, backlog, threads = hybrid
            check(lib().moert_model_create_hybrid(ctypes.byref(model.cfg.c()), ctypes.byref(model.weights()),
                                                  max_len, attn_splits, int(slots), int(backlog), int(threads),
                                                  ctypes.byref(h)))
        elif cache_slots is None:
            check(lib().moert_model_create(ctypes.byref(model.cfg.c()), ctypes.byref(model.weights()), max_len,
                                           attn_splits, ctypes.byref(h)))
        else:
            check(lib().moert_model_create_cached(ctypes.byref(model.cfg.c()), ctypes.byref(model.weights()),
                                                  max_len, attn_splits, int(cache_slots), ctypes.byref(h)))
        self.h = h

    def cache_stats(self):
        """(hits, copies) of the expert cache since creation or the last clear."""
        hi, co = ctypes.c_ulonglong(0), ctypes.c_ulonglong(0)
        check(lib().moert_cache_stats(self.h, ctypes.byref(hi), ctypes.byref(co)))
        return hi.value, co.value

    def cache_clear(self):
        check(lib().moert_cache_clear(self.h))

    def cache_fill(self):
        """Copies every expert not yet in the pool into its free slots, in key order, evicting nothing
        (ExpertCache::fill); returns the number copied."""
        n = ctypes.c_int(0)
        check(lib().moert_cache_fill(self.h, ctypes.byref(n)))
        return n.value

    def cache_prefetch(self, layer, experts):
        """Brings `experts` of `layer` into the pool ahead of a step (one tick of the LRU rule); returns the
        number that were not in the pool."""
        e = np.ascontiguousarray(experts, np.int32)
        n = ctypes.c_int(0)
        check(lib().moert_cache_prefetch(self.h, int(layer), ptr(e), len(e), ctypes.byref(n)))
        return n.value

    def cache_prefetch_mode(self, on: bool):
        """Prefetch branch inside the cached step (predicted experts copied while the attention half runs)."""
        check(lib().moert_cache_prefetch_mode(self.h, 1 if on else 0))

    def cache_predictions(self, pos0: int, n: int) -> np.ndarray:
        """Experts predicted by the prefetch branch: [n, layers, top_k] (-1 where none was recorded)."""
        c = self.cfg
        out = np.empty((n, c.layers, 8), np.int32)
        check(lib().moert_cache_predictions(self.h, pos0, n, ptr(out)))
        return out[:, :, :c.top_k]

    def cache_token_counts(self, pos0: int, n: int, words: int = 3) -> np.ndarray:
        """Per position and layer: [n, layers, words] = hits, copies inside the step, prefetched copies (hybrid: hits,
        admissions, admissions refused, requests computed on the host)."""
        out = np.empty((n, self.cfg.layers, 4), np.int32)
        check(lib().moert_cache_token_counts(self.h, pos0, n, ptr(out)))
        return out[:, :, :words]

    def attach_metrics(self, mx: Optional["Metrics"], interval_ms: int = 500):
        """Lets generate() fill and publish `mx` (None detaches); the publisher must outlive the attachment."""
        check(lib().moert_model_attach_metrics(self.h, mx.h if mx is not None else None, interval_ms))
        self._mx = mx

    def cache_counters(self) -> dict:
        c = moert_cache_counters()
        check(lib().moert_cache_counters_get(self.h, ctypes.byref(c)))
        return {n: getattr(c, n) for n, _ in moert_cache_counters._fields_}

    def close(self):
        if self.h:
            lib().moert_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def step(self, token: int, want_logits: bool = True):
        """One token: (logits, route ids [layers, k], route weights [layers, k], argmax) (GpuModel::step)."""
        c = self.cfg
        lg = np.empty(c.vocab, np.float32) if want_logits else None
        ids = np.empty((c.layers, c.top_k), np.int32)
        w = np.empty((c.layers, c.top_k), np.float32)
        am = ctypes.c_int(0)
        check(lib().moert_decode_step(self.h, int(token), ptr(lg), ptr(ids), ptr(w), ctypes.byref(am)))
        return lg, ids, w, am.value

    def batched_mode(self, mode: int):
        """0: multi-position steps with the per-row FMA kernels (bit-identical to decode steps); 1: experts through the
        grouped int8 MFMA kernels."""
        check(lib().moert_batched_mode(self.h, int(mode)))

    def step_batched(self, tokens, want_logits: bool = True):
        """Up to 32 tokens in one multi-position step: (logits of the last position, its argmax)
        (begin_step_tokens + the model step over m positions)."""
        t = np.ascontiguousarray(tokens, np.int32)
        lg = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        am = ctypes.c_int(0)
        check(lib().moert_step_batched(self.h, ptr(t), t.size, ptr(lg), ctypes.byref(am)))
        return lg, am.value

    def prefill(self, tokens, want_logits: bool = True):
        """Any number of tokens in blocks of at most 32 positions (le_ids): (last logits, last argmax)."""
        t = np.ascontiguousarray(tokens, np.int32)
        lg = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        am = ctypes.c_int(0)
        check(lib().moert_prefill(self.h, ptr(t), t.size, ptr(lg), ctypes.byref(am)))
        return lg, am.value

    def generate(self, prompt, n_new: int, gaps: bool = False):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_new, np.int32)
        g = np.empty(n_new, np.float32) if gaps else None
        check(lib().moert_generate(self.h, ptr(p), p.size, n_new, ptr(out), ptr(g)))
        return (out, g) if gaps else out

    def reset(self):
        check(lib().moert_reset_sequence(self.h))

    def set_position(self, pos: int):
        check(lib().moert_set_position(self.h, pos))

    def position(self) -> int:
        p = ctypes.c_int(0)
        check(lib().moert_get_position(self.h, ctypes.byref(p)))
        return p.value

    def kv_prefill(self, layer: int, k: np.ndarray, v: np.ndarray):
        """k, v: fp16 bits [kv_heads, n, head_dim]."""
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        check(lib().moert_kv_prefill_fp16(self.h, layer, ptr(k), ptr(v), k.shape[1]))

    def read_kv(self, layer: int, n: int):
        c = self.cfg
        k = np.empty((c.kv_heads, n, c.head_dim), np.uint16)
        v = np.empty_like(k)
        check(lib().moert_read_kv_fp16(self.h, layer, ptr(k), ptr(v), n))
        return k, v

    def hidden(self) -> np.ndarray:
        out = np.empty(self.cfg.hidden, np.float32)
        check(lib().moert_read_hidden(self.h, ptr(out)))
        return out

    def read_logits(self) -> np.ndarray:
        """Logits of the last step (Dense::read_logits)."""
        out = np.empty(self.cfg.vocab, np.float32)
        check(lib().moert_read_logits(self.h, ptr(out)))
        return out

    def time_steps(self, warmup: int, iters: int) -> float:
        ms = ctypes.c_double(0)
        check(lib().moert_time_steps(self.h, warmup, iters, ctypes.byref(ms)))
        return ms.value

    def timeline_step(self):
        """One step with per-workgroup phase stamps (libmoert_tl.so only): (records [launches, 1024, 12] u64,
        kinds [launches], layers [launches])."""
        n_max = 3 + 6 * self.cfg.layers
        out = np.zeros((n_max, 1024, TL_WORDS), np.uint64)
        kinds = np.zeros(n_max, np.int32)
        layers = np.zeros(n_max, np.int32)
        n = ctypes.c_int(0)
        check(lib().moert_timeline_step(self.h, ptr(out), ptr(kinds), ptr(layers), n_max, ctypes.byref(n)))
        return out[:n.value], kinds[:n.value], layers[:n.value]

    def time_kernel(self, kind: int, iters: int):
        us, n = ctypes.c_double(0), ctypes.c_int(0)
        check(lib().moert_time_kernel(self.h, kind, iters, ctypes.byref(us), ctypes.byref(n)))
        return us.value, n.value

    def kernel_path(self) -> str:
        """The decode step's kernels (moert_model_path): "layer" (each layer one launch), "fused" (the attention
        block and the MoE kernel over the XCDs), "block" (the attention block with the two-kernel MoE half) or
        "unfused"."""
        y, a, x = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
        check(lib().moert_model_path(self.h, ctypes.byref(y), ctypes.byref(a), ctypes.byref(x)))
        if y.value:
            return "layer"
        if a.value:
            return "fused" if x.value else "block"
        return "unfused"

    def fault_inject(self, bits: int):
        """Test hook: the fused kernels' waits named by `bits` (2 queries / K/V row, 4 split partials, 8 act vector;
        16 alone: the cache prefetch's copy wait) give up in the following launches, which still end normally
        (moert_fault_inject)."""
        check(lib().moert_fault_inject(self.h, bits))


# ---- checkpoints ------------------------------------------------------------------------------------------------
def config_from_json_native(text: str) -> Config:
    """Config::from_json (model.rs:34-61) through the library's parser."""
    b = text.encode()
    c = moert_config()
    check(lib().moert_config_from_json(b, len(b), ctypes.byref(c)))
    return Config(**{n: getattr(c, n) for n, _ in moert_config._fields_})


class Checkpoint:
    """Index of the *.safetensors files of a directory (Checkpoint::open, weights.rs:52-106); tensors read on
    demand (Checkpoint::bf16, weights.rs:109-122)."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(lib().moert_checkpoint_open(str(path).encode(), ctypes.byref(h)))
        self.h = h

    def tensor(self, name: str):
        """(dtype, shape) of a tensor."""
        dt = ctypes.create_string_buffer(32)
        shape = np.zeros(8, np.uint64)
        nd = ctypes.c_int(0)
        check(lib().moert_checkpoint_tensor(self.h, name.encode(), dt, 32, ptr(shape), 8, ctypes.byref(nd)))
        return dt.value.decode(), tuple(int(d) for d in shape[:nd.value])

    def bf16(self, name: str) -> np.ndarray:
        """The BF16 bits of a tensor, shaped."""
        _, shape = self.tensor(name)
        out = np.empty(int(np.prod(shape, dtype=np.uint64)) if shape else 1, np.uint16)
        check(lib().moert_checkpoint_read_bf16(self.h, name.encode(), ptr(out), out.size))
        return out.reshape(shape)

    def close(self):
        if self.h:
            lib().moert_checkpoint_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LoadedModel:
    """HostModel::load (model.rs:100-132) from a checkpoint, each BF16 matrix quantised on load to wdtype (the tied
    embedding / head to embed_dtype); usable wherever a SynthModel is (GpuModel, the oracle's CpuSession)."""

    def __init__(self, ck: Checkpoint, cfg: Config, wdtype: int = Q8_0, embed_dtype: int = Q8_0):
        h = ctypes.c_void_p()
        check(lib().moert_checkpoint_load(ck.h, ctypes.byref(cfg.c()), wdtype, embed_dtype, ctypes.byref(h)))
        self.h, self.cfg, self.wdtype, self.embed_dtype = h, cfg, wdtype, embed_dtype

    def weights(self) -> moert_model_weights:
        return lib().moert_host_model_weights(self.h).contents

    def close(self):
        if self.h:
            lib().moert_host_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def write_safetensors(path: str, tensors):
    """A safetensors file from (name, dtype string, shape, raw bytes) entries (the reference's test writer,
    tests/common/mod.rs:103-118, restated)."""
    import json
    head, data = {}, bytearray()
    for name, dt, shape, raw in tensors:
        start = len(data)
        data += raw
        head[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [start, len(data)]}
    h = json.dumps(head).encode()
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little") + h + bytes(data))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> BF16 bits, round to nearest even (bf16::from_f32)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def kv_prefill_data(cfg: Config, seed: int, layer: int, n: int):
    """fp16 N(0, 1) K and V of n positions for one layer, [kv_heads, n, head_dim] (the long-context workload)."""
    cnt = cfg.kv_heads * n * cfg.head_dim
    k = synth_fp16(seed, 50000 + 2 * layer, cnt).reshape(cfg.kv_heads, n, cfg.head_dim)
    v = synth_fp16(seed, 50001 + 2 * layer, cnt).reshape(cfg.kv_heads, n, cfg.head_dim)
    return k, v


class GpuBlock:
    """One MoE block, all experts resident (GpuLayer, gpu.rs:368-541)."""

    def __init__(self, hidden, inter, experts, top_k, router, gate_up, down, dtype=Q8_0, router_bias=None):
        self._keep = (router, gate_up, down, router_bias)
        self.hidden, self.top_k = hidden, top_k
        h = ctypes.c_void_p()
        check(lib().moert_block_create(hidden, inter, experts, top_k, ctypes.byref(moert_tensor(router.ctypes.data, dtype)),
                                       ptr(router_bias), ctypes.byref(moert_tensor(gate_up.ctypes.data, dtype)),
                                       ctypes.byref(moert_tensor(down.ctypes.data, dtype)), ctypes.byref(h)))
        self.h = h

    def forward(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(self.hidden, np.float32)
        ids = np.empty(self.top_k, np.int32)
        w = np.empty(self.top_k, np.float32)
        check(lib().moert_block_forward(self.h, ptr(x), ptr(y), ptr(ids), ptr(w)))
        return y, ids, w

    def time(self, iters: int) -> float:
        us = ctypes.c_double(0)
        check(lib().moert_block_time(self.h, iters, ctypes.byref(us)))
        return us.value

    def forward_batched(self, x: np.ndarray):
        """m positions at once (grouped MFMA experts): (y [m, H], ids [m, k], weights [m, k])."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.hidden)
        m = x.shape[0]
        y = np.empty((m, self.hidden), np.float32)
        ids = np.empty((m, self.top_k), np.int32)
        w = np.empty((m, self.top_k), np.float32)
        check(lib().moert_block_forward_batched(self.h, m, ptr(x), ptr(y), ptr(ids), ptr(w)))
        return y, ids, w

    def experts_in_step(self) -> int:
        n = ctypes.c_int(0)
        check(lib().moert_block_experts_in_step(self.h, ctypes.byref(n)))
        return n.value

    def batched_kernel(self, mode: int):
        """0: the batched step as four kernels; 1: as one launch over the XCDs (moert_block_batched_kernel)."""
        check(lib().moert_block_batched_kernel(self.h, int(mode)))
        self.fused = int(mode)

    def fault_inject(self, bits: int):
        """Test hook of the one-launch step: the waits named by `bits` (1 logits, 2 act vectors, 4 expert outputs,
        8 input codes) give up in the following steps, which still end normally (moert_block_fault_inject)."""
        check(lib().moert_block_fault_inject(self.h, bits))

    def close(self):
        if self.h:
            lib().moert_block_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def time_batched(blocks, m: int, iters: int):
    """Mean microseconds of one batched block step over `blocks` in turn, and of its four kernels."""
    arr = (ctypes.c_void_p * len(blocks))(*[b.h.value if isinstance(b.h, ctypes.c_void_p) else b.h for b in blocks])
    us = (ctypes.c_double * 5)()
    check(lib().moert_block_time_batched(arr, len(blocks), m, iters, us))
    if getattr(blocks[0], "fused", 0):
        return {"step": us[0], "launch": us[1]}
    return {"step": us[0], "route": us[1], "up": us[2], "down": us[3], "combine": us[4]}


def zipf_bias(experts: int, seed: int, s: float = 1.1) -> np.ndarray:
    """Router bias b_e = -s * ln(rank_e) over a seeded permutation of the experts (Zipf-skewed expert loads)."""
    rng = np.random.default_rng(seed)
    rank = np.empty(experts, np.int64)
    rank[rng.permutation(experts)] = np.arange(1, experts + 1)
    return (-s * np.log(rank)).astype(np.float32)


# ---- unit-parity entry points ------------------------------------------------------------------------------------
def router_topk(logits: np.ndarray, k: int):
    l = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    check(lib().moert_router_topk(ptr(l), l.size, k, ptr(ids), ptr(w)))
    return ids, w


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, np.float32)
    i = ctypes.c_int(0)
    check(lib().moert_argmax(ptr(v), v.size, ctypes.byref(i)))
    return i.value


def gemv(w: np.ndarray, dtype: int, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    check(lib().moert_gemv(ctypes.byref(moert_tensor(w.ctypes.data, dtype)), rows, cols, ptr(x), ptr(y)))
    return y


def dequant(w: np.ndarray, dtype: int, rows: int, cols: int) -> np.ndarray:
    out = np.empty(rows * cols, np.float32)
    check(lib().moert_dequant(ctypes.byref(moert_tensor(w.ctypes.data, dtype)), rows, cols, ptr(out)))
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    check(lib().moert_rmsnorm(ptr(x), ptr(w), x.size, eps, ptr(out)))
    return out


def rope(x: np.ndarray, head_dim: int, theta: float, pos: int) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy()
    check(lib().moert_rope(ptr(y), y.size // head_dim, head_dim, theta, pos))
    return y


def attn_decode(q, k_cache, v_cache, heads, kv_heads, max_len, length, scale, tiles_per_split):
    q = np.ascontiguousarray(q, np.float32)
    k_cache = np.ascontiguousarray(k_cache, np.uint16)
    v_cache = np.ascontiguousarray(v_cache, np.uint16)
    out = np.empty(heads * 64, np.float32)
    check(lib().moert_attn_decode(ptr(q), ptr(k_cache), ptr(v_cache), heads, kv_heads, 64, max_len, length, scale,
                                  tiles_per_split, ptr(out)))
    return out


def attn_decode_noalloc(q_dev: int, k_dev: int, v_dev: int, heads, kv_heads, max_len, length, scale,
                        tiles_per_split, out_dev: int, stream: int = 0) -> None:
    """moert_attn_decode on the caller's device buffers (raw device addresses), enqueued on `stream` (a hipStream_t
    address, 0 = default stream), with the split partials in the library's fixed scratch: no allocation."""
    check(lib().moert_attn_decode_noalloc(ctypes.c_void_p(q_dev), ctypes.c_void_p(k_dev), ctypes.c_void_p(v_dev),
                                          heads, kv_heads, 64, max_len, length, scale, tiles_per_split,
                                          ctypes.c_void_p(out_dev), ctypes.c_void_p(stream)))


def exp_device(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    check(lib().moert_exp_device(ptr(x), ptr(y), x.size))
    return y


def tiles_per_split(max_len: int, attn_splits: int) -> int:
    """64-position tiles per attention split when a cache of max_len positions is cut into at most attn_splits."""
    return (max_len // 64 + attn_splits - 1) // attn_splits


def attn_splits_for(max_len: int, tps: int) -> int:
    """Number of attention splits of tps tiles covering max_len positions."""
    return ((max_len + 63) // 64 + tps - 1) // tps


def copy_probe(nbytes: int, iters: int = 10) -> float:
    """Mean microseconds of one device-to-device copy of nbytes (HBM bandwidth reference)."""
    us = ctypes.c_double()
    check(lib().moert_copy_probe(ctypes.c_size_t(nbytes), iters, ctypes.byref(us)))
    return us.value


def read_probe(nbytes: int, iters: int = 10) -> float:
    """Mean microseconds of one cold streaming read of nbytes from HBM (achievable read-bandwidth reference)."""
    us = ctypes.c_double()
    check(lib().moert_read_probe(ctypes.c_size_t(nbytes), iters, ctypes.byref(us)))
    return us.value


def h2d_probe(nbytes: int, iters: int = 5):
    """Mean microseconds of one pinned-host -> HBM copy of nbytes: (by a copy kernel, by hipMemcpyAsync)."""
    k, m = ctypes.c_double(), ctypes.c_double()
    check(lib().moert_h2d_probe(ctypes.c_size_t(nbytes), iters, ctypes.byref(k), ctypes.byref(m)))
    return k.value, m.value


def step_bytes(cfg: Config, wdtype: int, embed_dtype: int, context: int) -> int:
    """Algorithmic HBM bytes of one decode step at `context` cached positions (weights once, KV once)."""
    H, d, I = cfg.hidden, cfg.head_dim, cfg.inter
    qd, kvd = cfg.heads * d, cfg.kv_heads * d
    attn = dtype_bytes(wdtype, (qd + 2 * kvd) * H) + dtype_bytes(wdtype, H * qd)
    router = dtype_bytes(wdtype, cfg.experts * H)
    experts = cfg.top_k * (dtype_bytes(wdtype, 2 * I * H) + dtype_bytes(wdtype, H * I))
    norms = 2 * H * 4
    per_layer = attn + router + experts + norms
    kv = cfg.layers * 2 * kvd * 2 * context
    head = dtype_bytes(embed_dtype, cfg.vocab * H)
    return cfg.layers * per_layer + kv + head


# ---- runtime metrics (the reference's moe-monitor transport, rust/moe-monitor/src/snapshot.rs) ----
METRICS_SCHEMA = 1  # SCHEMA (snapshot.rs:14)
METRICS_STALE_MS = 3000  # STALE_MS (snapshot.rs:16)
STATE_IDLE, STATE_READING, STATE_GENERATING, STATE_QUEUED, STATE_ERROR = range(5)


class Metrics:
    """The native snapshot publisher (moert_metrics_*), as Publisher + Snapshot (snapshot.rs:18-185): sections set
    field by field, published atomically (temporary file + rename) to `path` (None: the default path)."""

    def __init__(self, path=None):
        h = ctypes.c_void_p()
        check(lib().moert_metrics_create(None if path is None else os.fsencode(path), ctypes.byref(h)))
        self.h = h.value

    @property
    def path(self) -> str:
        buf = ctypes.create_string_buffer(4096)
        check(lib().moert_metrics_path(self.h, buf, len(buf)))
        return os.fsdecode(buf.value)

    def set_model(self, name, layers, experts, experts_per_tok):
        check(lib().moert_metrics_set_model(self.h, name.encode(), layers, experts, experts_per_tok))

    def set_state(self, kind, a=0, b=0, message=None):
        check(lib().moert_metrics_set_state(self.h, kind, a, b, None if message is None else message.encode()))

    def set_speed(self, **kw):
        check(lib().moert_metrics_set_speed(self.h, ctypes.byref(moert_metrics_speed(**kw))))

    def set_context(self, used, max_):
        check(lib().moert_metrics_set_context(self.h, used, max_))

    def set_cache(self, **kw):
        check(lib().moert_metrics_set_cache(self.h, ctypes.byref(moert_metrics_cache(**kw))))

    def set_window(self, **kw):
        check(lib().moert_metrics_set_window(self.h, ctypes.byref(moert_metrics_window(**kw))))

    def add_request(self, status="ok", **kw):
        r = moert_metrics_request(status=status.encode(), **kw)
        check(lib().moert_metrics_add_request(self.h, ctypes.byref(r)))

    def setting(self, key, value):
        check(lib().moert_metrics_setting(self.h, key.encode(), value.encode()))

    def event(self, level, message):
        check(lib().moert_metrics_event(self.h, level.encode(), message.encode()))

    def json(self) -> str:
        need = ctypes.c_size_t()
        check(lib().moert_metrics_json(self.h, None, 0, ctypes.byref(need)))
        buf = ctypes.create_string_buffer(need.value + 4096)
        check(lib().moert_metrics_json(self.h, buf, len(buf), ctypes.byref(need)))
        return buf.value.decode()

    def publish(self):
        check(lib().moert_metrics_publish(self.h))

    def close(self):
        if self.h:
            lib().moert_metrics_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def metrics_now_ms() -> int:
    return int(time.time() * 1000)


def read_metrics(path, now_ms=None):
    """What a monitor knows of the runtime from one read of the file (snapshot::read, snapshot.rs:187-215):
    ("absent", None) without a file, ("invalid", message) for unreadable JSON or another schema, ("stale", snap)
    after METRICS_STALE_MS without a publication, else ("live", snap)."""
    now_ms = metrics_now_ms() if now_ms is None else now_ms
    try:
        raw = open(path, "rb").read()
    except FileNotFoundError:
        return "absent", None
    except OSError as e:
        return "invalid", str(e)
    try:
        snap = json.loads(raw)
    except ValueError as e:
        return "invalid", f"invalid JSON: {e}"
    if not isinstance(snap, dict) or snap.get("schema") != METRICS_SCHEMA:
        return "invalid", f"schema {snap.get('schema') if isinstance(snap, dict) else None} " \
                          f"(the monitor knows {METRICS_SCHEMA})"
    age = max(0, now_ms - int(snap.get("ts_ms", 0)))
    return ("stale" if age > METRICS_STALE_MS else "live"), snap


# ---- expert placement of the host-CPU hybrid (the D1 service line in its deterministic mode) ----
PLACEMENT_FIELDS = ("needed", "hits", "cpu", "copies", "dropped", "deferred")


class Placement:
    """moert_placement_*: the table / LFU admission / held-copy state machine of the hybrid, stepped on routes."""

    def __init__(self, layers, experts, top_k, slots, backlog):
        h = ctypes.c_void_p()
        check(lib().moert_placement_create(layers, experts, top_k, slots, backlog, ctypes.byref(h)))
        self.h, self.L, self.E, self.k = h.value, layers, experts, top_k

    def step(self, ids):
        """ids [layers][m][top_k]; returns (requests served on the GPU, copies queued)."""
        a = np.ascontiguousarray(ids, np.int32)
        assert a.ndim == 3 and a.shape[0] == self.L and a.shape[2] == self.k, a.shape
        g, c = ctypes.c_int(), ctypes.c_int()
        check(lib().moert_placement_step(self.h, ptr(a), a.shape[1], ctypes.byref(g), ctypes.byref(c)))
        return g.value, c.value

    def counters(self) -> dict:
        c = moert_cache_counters()
        check(lib().moert_placement_counters(self.h, ctypes.byref(c)))
        return {n: getattr(c, n) for n in PLACEMENT_FIELDS}

    def table(self) -> np.ndarray:
        t = np.empty(self.L * self.E, np.int32)
        check(lib().moert_placement_table(self.h, ptr(t)))
        return t

    def close(self):
        if self.h:
            lib().moert_placement_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Freq:
    """moert_freq_*: the decayed frequency of the LFU admission."""

    def __init__(self, keys, layers):
        h = ctypes.c_void_p()
        check(lib().moert_freq_create(keys, layers, ctypes.byref(h)))
        self.h = h.value

    def touch(self, key, step):
        check(lib().moert_freq_touch(self.h, key, step))

    def score(self, key) -> float:
        v = ctypes.c_double()
        check(lib().moert_freq_score(self.h, key, ctypes.byref(v)))
        return v.value

    def clear(self):
        check(lib().moert_freq_clear(self.h))

    def __del__(self):
        if getattr(self, "h", None):
            lib().moert_freq_destroy(self.h)
            self.h = None


# ---- tokenizer (tokenizador.rs) ----
ROLE_SYSTEM, ROLE_USER, ROLE_ASSISTANT = 0, 1, 2


class Tokenizer:
    """moert_tokenizer_*: the byte-level BPE of a Granite tokenizer.json (Tokenizador)."""

    def __init__(self, path=None, json_text=None):
        h = ctypes.c_void_p()
        if json_text is not None:
            raw = json_text.encode() if isinstance(json_text, str) else bytes(json_text)
            check(lib().moert_tokenizer_from_json(raw, len(raw), ctypes.byref(h)))
        else:
            check(lib().moert_tokenizer_load(os.fsencode(path), ctypes.byref(h)))
        self.h = h.value

    def vocab_size(self) -> int:
        n = ctypes.c_int()
        check(lib().moert_tokenizer_vocab_size(self.h, ctypes.byref(n)))
        return n.value

    def encode(self, text: str) -> List[int]:
        raw = text.encode()
        out = np.empty(max(1, len(raw)), np.uint32)
        n = ctypes.c_size_t()
        check(lib().moert_tokenizer_encode(self.h, raw, len(raw), ptr(out), out.size, ctypes.byref(n)))
        return [int(v) for v in out[:n.value]]

    def decode_bytes(self, ids) -> bytes:
        a = np.ascontiguousarray(ids, np.uint32)
        n = ctypes.c_size_t()
        check(lib().moert_tokenizer_decode(self.h, ptr(a), a.size, 0, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value + 1)
        check(lib().moert_tokenizer_decode(self.h, ptr(a), a.size, 0, buf, len(buf), ctypes.byref(n)))
        return buf.raw[:n.value]

    def decode(self, ids) -> str:
        a = np.ascontiguousarray(ids, np.uint32)
        n = ctypes.c_size_t()
        check(lib().moert_tokenizer_decode(self.h, ptr(a), a.size, 1, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value + 1)
        check(lib().moert_tokenizer_decode(self.h, ptr(a), a.size, 1, buf, len(buf), ctypes.byref(n)))
        return buf.raw[:n.value].decode()

    def close(self):
        if self.h:
            lib().moert_tokenizer_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pretokenize(text: str) -> List[str]:
    """The GPT-2 pattern's pieces of `text` (pre_tokeniza)."""
    raw = text.encode()
    n = ctypes.c_size_t()
    check(lib().moert_tokenizer_pretokenize(raw, len(raw), None, 0, ctypes.byref(n)))
    ends = np.empty(max(1, n.value), np.uint64)
    check(lib().moert_tokenizer_pretokenize(raw, len(raw), ptr(ends), ends.size, ctypes.byref(n)))
    out, s = [], 0
    for e in ends[:n.value]:
        out.append(raw[s:int(e)].decode())
        s = int(e)
    return out


def chat_render(messages, add_generation_prompt=True, date="") -> str:
    """messages: [(role, content)] with roles ROLE_*; the fixed Granite 3.1 chat template (renderiza_chat)."""
    n = len(messages)
    roles = (ctypes.c_int * max(1, n))(*[r for r, _ in messages])
    contents = (ctypes.c_char_p * max(1, n))(*[c.encode() for _, c in messages])
    need = ctypes.c_size_t()
    check(lib().moert_chat_render(roles, contents, n, int(add_generation_prompt), date.encode(), None, 0,
                                  ctypes.byref(need)))
    buf = ctypes.create_string_buffer(need.value + 1)
    check(lib().moert_chat_render(roles, contents, n, int(add_generation_prompt), date.encode(), buf, len(buf),
                                  ctypes.byref(need)))
    return buf.raw[:need.value].decode()


def format_date(year, month, day) -> str:
    buf = ctypes.create_string_buffer(64)
    check(lib().moert_format_date(year, month, day, buf, len(buf)))
    return buf.value.decode()
