"""ctypes wrapper of the oracle (oracle/liboracle.so) — test infrastructure only.

Imported by tests/, by __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg; never by the
product package. The C++ restatement it wraps follows rust/moe-rt/src/{model.rs,block.rs,cpu.rs,pool.rs} and the
split-KV attention of gpu.rs:205-292 (see oracle.h for the evaluation order).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i, f, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
        sig = {
            "orc_exp": (f, [f]),
            "orc_exp_n": (None, [vp, vp, sz]),
            "orc_h2f_n": (None, [vp, vp, sz]),
            "orc_f2h_n": (None, [vp, vp, sz]),
            "orc_dequant": (None, [vp, i, sz, vp]),
            "orc_dot": (f, [vp, i, i, sz, vp]),
            "orc_gemv": (None, [vp, i, i, i, vp, vp, i]),
            "orc_rmsnorm": (None, [vp, vp, i, f, vp]),
            "orc_rope_cos_sin": (None, [f, i, i, vp]),
            "orc_rope": (None, [vp, i, i, vp]),
            "orc_route": (None, [vp, vp, i, i, vp, vp]),
            "orc_swiglu": (None, [vp, i, vp]),
            "orc_moe_norm_route": (None, [vp, vp, vp, vp, i, i, f, vp, vp]),
            "orc_argmax": (i, [vp, i]),
            "orc_moe_block": (None, [i, i, i, i, vp, vp, vp, vp, vp, vp, vp, vp, i]),
            "orc_attention": (None, [vp, vp, vp, i, i, i, i, i, f, i, vp]),
            "orc_tiles_per_split": (i, [i, i]),
            "orc_experts_step": (None, [i, i, i, i, vp, vp, vp, vp, vp, vp, i]),
            "orc_quant_hilo": (None, [vp, i, vp, vp, vp]),
            "orc_dot_hilo": (f, [vp, i, i, sz, vp, vp, vp]),
            "orc_experts_grouped": (None, [i, i, i, i, vp, vp, vp, vp, vp, vp, i]),
            "orc_moe_block_batched": (None, [i, i, i, i, vp, vp, vp, vp, i, vp, vp, vp, vp, i]),
            "orc_lru_replay": (None, [vp, i, i, i, i, i, vp]),
            "orc_lru_create": (vp, [i, i, i]),
            "orc_lru_destroy": (None, [vp]),
            "orc_lru_step_layer": (None, [vp, i, vp, i]),
            "orc_lru_prefetch": (i, [vp, i, vp, i]),
            "orc_lru_fill": (i, [vp]),
            "orc_lru_stats": (None, [vp, vp]),
            "orc_lru_slots": (None, [vp, vp]),
            "orc_session_create": (i, [vp, vp, i, i, i, ctypes.POINTER(vp)]),
            "orc_session_destroy": (None, [vp]),
            "orc_session_step": (i, [vp, i, vp, vp, vp, vp]),
            "orc_session_set_pos": (None, [vp, i]),
            "orc_session_pos": (i, [vp]),
            "orc_session_kv_prefill": (i, [vp, i, vp, vp, i]),
            "orc_session_read_kv": (i, [vp, i, vp, vp, i]),
            "orc_dot_hilo_quarters": (f, [vp, i, i, sz, vp, vp, vp]),
            "orc_rmsnorm_threads": (None, [vp, vp, i, f, i, vp]),
            "orc_session_step_grouped": (i, [vp, vp, i, vp, vp, vp, vp]),
            "port_session_create": (i, [vp, vp, i, i, ctypes.POINTER(vp)]),
            "port_session_destroy": (None, [vp]),
            "port_session_set_pos": (None, [vp, i]),
            "port_session_kv_prefill": (i, [vp, i, vp, vp, i]),
            "port_session_step": (i, [vp, i, vp, vp, vp]),
            "port_dot": (f, [vp, i, i, sz, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def exp(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_exp_n(_p(x), _p(y), x.size)
    return y


def h2f(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_h2f_n(_p(h), _p(out), h.size)
    return out


def f2h(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f2h_n(_p(x), _p(out), x.size)
    return out


def dequant(w, dtype, n):
    out = np.empty(n, np.float32)
    lib().orc_dequant(_p(w), dtype, n, _p(out))
    return out


def dot(w, dtype, cols, row, x):
    return float(lib().orc_dot(_p(w), dtype, cols, row, _p(_f32(x))))


def gemv(w, dtype, rows, cols, x, threads=4):
    y = np.empty(rows, np.float32)
    lib().orc_gemv(_p(w), dtype, rows, cols, _p(_f32(x)), _p(y), threads)
    return y


def rmsnorm(x, w, eps):
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), _p(w), x.size, eps, _p(out))
    return out


def rope_cos_sin(theta, head_dim, pos):
    cs = np.empty(head_dim, np.float32)
    lib().orc_rope_cos_sin(theta, head_dim, pos, _p(cs))
    return cs


def rope(x, head_dim, cs):
    y = _f32(x).copy()
    lib().orc_rope(_p(y), y.size, head_dim, _p(_f32(cs)))
    return y


def route(logits, k, bias=None):
    l = _f32(logits)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    lib().orc_route(_p(l), _p(None if bias is None else _f32(bias)), l.size, k, _p(ids), _p(w))
    return ids, w


def moe_norm_route(h, lnw, router, dtype, experts, eps, bias=None):
    """The MoE half's rmsnorm and router logits in the engine's partial-block order: (xn, logits)."""
    mt = _moert()
    h, lnw = _f32(h), _f32(lnw)
    r = mt.moert_tensor(router.ctypes.data, dtype)
    xn = np.empty_like(h)
    lg = np.empty(experts, np.float32)
    lib().orc_moe_norm_route(_p(h), _p(lnw), ctypes.byref(r), _p(None if bias is None else _f32(bias)), h.size,
                             experts, eps, _p(xn), _p(lg))
    return xn, lg


def swiglu(h):
    h = _f32(h)
    a = np.empty(h.size // 2, np.float32)
    lib().orc_swiglu(_p(h), h.size // 2, _p(a))
    return a


def argmax(v):
    v = _f32(v)
    return int(lib().orc_argmax(_p(v), v.size))


def _moert():
    import importlib
    import sys
    pkg = os.path.join(os.path.dirname(_HERE), "lastro-rust_amd")
    if pkg not in sys.path:
        sys.path.insert(0, pkg)
    return importlib.import_module("moert")


def moe_block(hidden, inter, experts, k, router, gate_up, down, dtype, x, bias=None, threads=4):
    mt = _moert()
    r, gu, dn = (mt.moert_tensor(a.ctypes.data, dtype) for a in (router, gate_up, down))
    x = _f32(x)
    y = np.empty(hidden, np.float32)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    lib().orc_moe_block(hidden, inter, experts, k, ctypes.byref(r), _p(None if bias is None else _f32(bias)),
                        ctypes.byref(gu), ctypes.byref(dn), _p(x), _p(y), _p(ids), _p(w), threads)
    return y, ids, w


def attention(q, k_cache, v_cache, heads, kv_heads, max_len, length, scale, tiles_per_split):
    q = _f32(q)
    kc = np.ascontiguousarray(k_cache, np.uint16)
    vc = np.ascontiguousarray(v_cache, np.uint16)
    out = np.empty(heads * 64, np.float32)
    lib().orc_attention(_p(q), _p(kc), _p(vc), heads, kv_heads, 64, max_len, length, scale, tiles_per_split, _p(out))
    return out


def tiles_per_split(max_len, attn_splits):
    return int(lib().orc_tiles_per_split(max_len, attn_splits))


def experts_step(hidden, inter, m, k, gate_up, down, dtype, x, ids, weights, threads=4):
    mt = _moert()
    gu, dn = mt.moert_tensor(gate_up.ctypes.data, dtype), mt.moert_tensor(down.ctypes.data, dtype)
    x = _f32(x)
    ids = np.ascontiguousarray(ids, np.int32)
    weights = _f32(weights)
    y = np.empty(m * hidden, np.float32)
    lib().orc_experts_step(hidden, inter, m, k, ctypes.byref(gu), ctypes.byref(dn), _p(x), _p(ids), _p(weights),
                           _p(y), threads)
    return y.reshape(m, hidden)


def quant_hilo(x):
    """15-bit block codes of x: (hi int8, lo int8, d f32 per 32-block) with x ~ (256*hi + lo) * d."""
    x = _f32(x)
    hi = np.empty(x.size, np.int8)
    lo = np.empty(x.size, np.int8)
    d = np.empty(x.size // 32, np.float32)
    lib().orc_quant_hilo(_p(x), x.size, _p(hi), _p(lo), _p(d))
    return hi, lo, d


def dot_hilo(w, dtype, cols, row, hi, lo, d):
    return float(lib().orc_dot_hilo(w.ctypes.data, dtype, cols, row, _p(hi), _p(lo), _p(d)))


def experts_grouped(hidden, inter, m, k, gate_up, down, dtype, x, ids, weights, threads=4):
    mt = _moert()
    gu, dn = mt.moert_tensor(gate_up.ctypes.data, dtype), mt.moert_tensor(down.ctypes.data, dtype)
    x = _f32(x)
    ids = np.ascontiguousarray(ids, np.int32)
    weights = _f32(weights)
    y = np.empty(m * hidden, np.float32)
    lib().orc_experts_grouped(hidden, inter, m, k, ctypes.byref(gu), ctypes.byref(dn), _p(x), _p(ids), _p(weights),
                              _p(y), threads)
    return y.reshape(m, hidden)


def moe_block_batched(hidden, inter, experts, k, router, gate_up, down, dtype, x, bias=None, threads=4):
    """m = len(x) // hidden positions through one MoE block in the grouped integer order: (y, ids, weights)."""
    mt = _moert()
    r, gu, dn = (mt.moert_tensor(a.ctypes.data, dtype) for a in (router, gate_up, down))
    x = _f32(x)
    m = x.size // hidden
    y = np.empty(m * hidden, np.float32)
    ids = np.empty(m * k, np.int32)
    w = np.empty(m * k, np.float32)
    lib().orc_moe_block_batched(hidden, inter, experts, k, ctypes.byref(r), _p(None if bias is None else _f32(bias)),
                                ctypes.byref(gu), ctypes.byref(dn), m, _p(x), _p(y), _p(ids), _p(w), threads)
    return y.reshape(m, hidden), ids.reshape(m, k), w.reshape(m, k)


def lru_replay(routes, experts, slots):
    """(hits, copies, cpu) of the LRU expert cache over routes [steps, layers, k] (C restatement)."""
    r = np.ascontiguousarray(routes, np.int32)
    steps, layers, k = r.shape
    out = np.zeros(3, np.uint64)
    lib().orc_lru_replay(_p(r), steps, layers, k, experts, slots, _p(out))
    return tuple(int(v) for v in out)


def lru_reference(routes, experts, cap):
    """The same rule written as rust/moe-rt/tests/model.rs:380-412 states it (list scans), for small traces:
    slots hold (key, last use) or None; the requested keys are touched first, then each missing key takes the
    first free slot or else the oldest slot used before this tick (first such on ties)."""
    slots = [None] * cap
    clock = hits = copies = cpu = 0
    for step in routes:
        for l, chosen in enumerate(step):
            clock += 1
            keys = [l * experts + int(e) for e in chosen]
            for i, s in enumerate(slots):
                if s is not None and s[0] in keys:
                    slots[i] = (s[0], clock)
            for key in keys:
                if any(s is not None and s[0] == key for s in slots):
                    hits += 1
                    continue
                victim = next((i for i, s in enumerate(slots) if s is None), None)
                if victim is None:
                    old = [(s[1], i) for i, s in enumerate(slots) if s[1] < clock]
                    victim = min(old)[1] if old else None
                if victim is None:
                    cpu += 1
                else:
                    slots[victim] = (key, clock)
                    copies += 1
    return hits, copies, cpu


class Lru:
    """The LRU expert cache as a state machine (orc_lru): decode-step layers (counted), prefetch ticks and fills
    (uncounted), for traces that mix them."""

    def __init__(self, layers, experts, slots):
        self.layers, self.experts, self.slots = layers, experts, slots
        self.h = lib().orc_lru_create(layers, experts, slots)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_lru_destroy(self.h)
            self.h = None

    def step(self, routes):
        """One decode step: routes [layers, k]."""
        r = np.ascontiguousarray(routes, np.int32)
        for l in range(r.shape[0]):
            lib().orc_lru_step_layer(self.h, l, _p(r[l]), r.shape[1])

    def prefetch(self, layer, ids):
        a = np.ascontiguousarray(ids, np.int32)
        return int(lib().orc_lru_prefetch(self.h, layer, _p(a), a.size))

    def fill(self):
        return int(lib().orc_lru_fill(self.h))

    def stats(self):
        out = np.zeros(3, np.uint64)
        lib().orc_lru_stats(self.h, _p(out))
        return tuple(int(v) for v in out)

    def slot_keys(self):
        out = np.empty(self.slots, np.int32)
        lib().orc_lru_slots(self.h, _p(out))
        return out


def lru_reference_ops(ops, experts, cap, fill_stamp_clock=True):
    """lru_reference over a trace of operations, for traces with fills and prefetches: ("step", layer, ids) is a
    counted tick, ("prefetch", layer, ids) an uncounted one, ("fill", n_keys) puts every absent key in key order into
    the first free slot with the current clock (ExpertCache::fill -> copy_on_compute, cache.rs:212-227,
    cache/core.rs:366-377). fill_stamp_clock=False stamps 0 instead (a mutant the tests must tell apart)."""
    slots = [None] * cap
    clock = hits = copies = cpu = 0
    for op in ops:
        if op[0] == "fill":
            for key in range(op[1]):
                if any(s is not None and s[0] == key for s in slots):
                    continue
                free = next((i for i, s in enumerate(slots) if s is None), None)
                if free is None:
                    break
                slots[free] = (key, clock if fill_stamp_clock else 0)
            continue
        kind, l, chosen = op
        counted = kind == "step"
        clock += 1
        keys = [l * experts + int(e) for e in chosen]
        for i, s in enumerate(slots):
            if s is not None and s[0] in keys:
                slots[i] = (s[0], clock)
        for key in keys:
            if any(s is not None and s[0] == key for s in slots):
                hits += counted
                continue
            victim = next((i for i, s in enumerate(slots) if s is None), None)
            if victim is None:
                old = [(s[1], i) for i, s in enumerate(slots) if s[1] < clock]
                victim = min(old)[1] if old else None
            if victim is None:
                cpu += counted
            else:
                slots[victim] = (key, clock)
                copies += counted
    return hits, copies, cpu


class CpuSession:
    """CpuSession (rust/moe-rt/src/model.rs:160-243) over a moert.SynthModel, fp16 KV cache of max_len."""

    def __init__(self, model, max_len, attn_splits=64, threads=None):
        self.model, self.cfg = model, model.cfg
        threads = threads or min(16, os.cpu_count() or 1)
        self.threads = threads
        h = ctypes.c_void_p()
        rc = lib().orc_session_create(ctypes.byref(model.cfg.c()), ctypes.byref(model.weights()), max_len,
                                      attn_splits, threads, ctypes.byref(h))
        if rc != 0:
            raise RuntimeError(f"orc_session_create failed: {rc}")
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_session_destroy(self.h)
            self.h = None

    def step(self, token, want_logits=True):
        c = self.cfg
        lg = np.empty(c.vocab, np.float32) if want_logits else None
        ids = np.empty((c.layers, c.top_k), np.int32)
        w = np.empty((c.layers, c.top_k), np.float32)
        hid = np.empty(c.hidden, np.float32)
        rc = lib().orc_session_step(self.h, int(token), _p(lg), _p(ids), _p(w), _p(hid))
        if rc != 0:
            raise RuntimeError(f"orc_session_step failed: {rc}")
        return lg, ids, w, hid

    def step_grouped(self, tokens, want_logits=True):
        """The engine's grouped multi-position step (moert_batched_mode 1) over n <= 32 tokens: (last logits,
        routes [n, layers, k], weights [n, layers, k], last hidden state)."""
        c = self.cfg
        t = np.ascontiguousarray(tokens, np.int32)
        n = t.size
        lg = np.empty(c.vocab, np.float32) if want_logits else None
        ids = np.empty((n, c.layers, c.top_k), np.int32)
        w = np.empty((n, c.layers, c.top_k), np.float32)
        hid = np.empty(c.hidden, np.float32)
        rc = lib().orc_session_step_grouped(self.h, _p(t), n, _p(lg), _p(ids), _p(w), _p(hid))
        if rc != 0:
            raise RuntimeError(f"orc_session_step_grouped failed: {rc}")
        return lg, ids, w, hid

    def set_position(self, pos):
        lib().orc_session_set_pos(self.h, pos)

    def position(self):
        return int(lib().orc_session_pos(self.h))

    def kv_prefill(self, layer, k, v):
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        rc = lib().orc_session_kv_prefill(self.h, layer, _p(k), _p(v), k.shape[1])
        if rc != 0:
            raise RuntimeError(f"kv_prefill failed: {rc}")

    def read_kv(self, layer, n):
        c = self.cfg
        k = np.empty((c.kv_heads, n, c.head_dim), np.uint16)
        v = np.empty_like(k)
        lib().orc_session_read_kv(self.h, layer, _p(k), _p(v), n)
        return k, v

    def generate(self, prompt, n_new):
        """Greedy: prompt token by token, then n_new argmax tokens (m1b-gulosa.rs:85-105); also the top1-top2 gaps."""
        lg = None
        for t in prompt:
            lg, _, _, self.last_hidden = self.step(int(t))
        out, gaps = [], []
        for i in range(n_new):
            nxt = argmax(lg)
            s = np.sort(lg)
            gaps.append(float(s[-1] - s[-2]))
            out.append(nxt)
            if i + 1 < n_new:
                lg, _, _, self.last_hidden = self.step(nxt)
        self.last_logits = lg  # the logits the last token was chosen from
        return np.array(out, np.int32), np.array(gaps, np.float32)


class PortSession:
    """The CPU port of the reference's CPU decode path (cpu_port.cpp: CpuSession::step with dot_avx2's accumulation,
    an f32 KV cache and attention on the calling thread), timed as bench.py's CPU baseline."""

    def __init__(self, model, max_len, threads=None):
        self.model, self.cfg = model, model.cfg
        self.threads = threads or (os.cpu_count() or 1)
        h = ctypes.c_void_p()
        rc = lib().port_session_create(ctypes.byref(model.cfg.c()), ctypes.byref(model.weights()), max_len,
                                       self.threads, ctypes.byref(h))
        if rc != 0:
            raise RuntimeError(f"port_session_create failed: {rc}")
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib().port_session_destroy(self.h)
            self.h = None

    def step(self, token, want_logits=True):
        c = self.cfg
        lg = np.empty(c.vocab, np.float32) if want_logits else None
        ids = np.empty((c.layers, c.top_k), np.int32)
        w = np.empty((c.layers, c.top_k), np.float32)
        rc = lib().port_session_step(self.h, int(token), _p(lg), _p(ids), _p(w))
        if rc != 0:
            raise RuntimeError(f"port_session_step failed: {rc}")
        return lg, ids, w

    def set_position(self, pos):
        lib().port_session_set_pos(self.h, pos)

    def kv_prefill(self, layer, k, v):
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        rc = lib().port_session_kv_prefill(self.h, layer, _p(k), _p(v), k.shape[1])
        if rc != 0:
            raise RuntimeError(f"port kv_prefill failed: {rc}")


def port_dot(w: np.ndarray, dtype: int, cols: int, row: int, x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, np.float32)
    return float(lib().port_dot(_p(w), dtype, cols, row, _p(x)))


def dot_hilo_quarters(w, dtype, cols, row, hi, lo, d):
    return float(lib().orc_dot_hilo_quarters(_p(w), dtype, cols, row, _p(np.ascontiguousarray(hi, np.int8)),
                                             _p(np.ascontiguousarray(lo, np.int8)),
                                             _p(np.ascontiguousarray(d, np.float32))))


def rmsnorm_threads(h, lnw, eps, threads):
    h = np.ascontiguousarray(h, np.float32)
    lnw = np.ascontiguousarray(lnw, np.float32)
    out = np.empty_like(h)
    lib().orc_rmsnorm_threads(_p(h), _p(lnw), h.size, eps, threads, _p(out))
    return out
