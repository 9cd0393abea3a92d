"""One Gemma 4 decode step through the raw C ABI, in the order the reference's
graph makes its calls (src/gemma4/metal.rs:538-794, the routed experts
through the storage-backed cache at :972-1042), over a small GGUF v3 file
written and memory-mapped here (tests/gguf_file.py):

  per layer   rms_norm(attention_norm)  matvec_mapped q, k, v
              rms_norm per head (query_norm, key_norm, none for v)
              rope_neox_in_place q, k    append_kv    attention_cached
              matvec_mapped o            rms_norm(post_attention_norm)   add
              rms_norm(feed_forward_norm)  matvec_mapped gate, up  gelu_mul
              matvec_mapped down         rms_norm(shared_post_norm)
              rms_norm(routed_pre_norm)  rms_norm(no weight) * router_scale / sqrt(hidden)
              matvec_mapped router       top_k_softmax
              per selected expert: expert_acquire (with_expert) ->
                matvec_owned gate_up -> gelu_mul -> matvec_owned down ->
                expert_release; out = fma(expert, p * down_scale[e], out)
              rms_norm(routed_post_norm) add  rms_norm(post_feed_forward_norm)
              add   * layer_output_scale
  output      rms_norm(output_norm)  matvec_mapped output  softcap

Two layers, one sliding (a 3-position ring that wraps) and one full with
partial rotary dimensions, decode five tokens.  The expert cache is
file-backed (dmhip_expert_cache_new_file over the same GGUF) with two slots
per layer, so experts are read, evicted and read again.  Every library call
is checked against the oracle's restatement of the same operation on the
same inputs, and an independent oracle composition of the whole step gives
the hidden states, the selected experts (identical) and the logits."""
import ctypes
import math
import mmap
import os

import numpy as np
import pytest

from diskmule_amd import synth
from diskmule_amd.hip import load_library
from oracle import capi
from tests import gguf_file
from tests.exact import fma32
from tests.tolerance import assert_close

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0, F16, F32 = 12, 14, 8, 1, 0
HIDDEN, QH, KVH, HD, VOCAB = 256, 4, 2, 64, 1000
FFN, EXPERTS, USED, EXPERT_WIDTH = 512, 8, 2, 128
EPS, SOFTCAP, WINDOW, MAX_CONTEXT = 1e-6, 30.0, 3, 16
LAYERS = [  # (sliding, rotated pairs, theta)
    (True, 32, 10000.0),
    (False, 16, 1000000.0),
]
TOKENS = [17, 503, 4, 999, 250]

f32p = ctypes.POINTER(ctypes.c_float)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _tensors():
    """(name, dims, type, bytes) of the small model, and name -> encoded."""
    t, enc = [], {}

    def add(name, dims, kind, seed, scale=1.0):
        if kind in (F32, F16):
            n = int(np.prod(dims))
            v = (synth.normal(synth.activation_seed(700, seed), n) * np.float32(scale)).astype(np.float32)
            data = v if kind == F32 else v.astype(np.float16)
            raw = data.view(np.uint8)
        else:
            cols, rows = dims[0], int(np.prod(dims[1:]))
            raw = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(700, seed))
        t.append((name, list(dims), kind, raw.tobytes()))
        enc[name] = raw

    add("token_embd.weight", [HIDDEN, VOCAB], F32, 1, 0.05)
    for l in range(len(LAYERS)):
        s = 100 * (l + 1)
        for i, n in enumerate(("attn_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm_1", "pre_ffw_norm_2",
                               "post_ffw_norm_2", "post_ffw_norm")):
            add(f"blk.{l}.{n}.weight", [HIDDEN], F32, s + i, 0.2)
        add(f"blk.{l}.attn_q.weight", [HIDDEN, QH * HD], Q4_K, s + 10)
        add(f"blk.{l}.attn_k.weight", [HIDDEN, KVH * HD], Q4_K, s + 11)
        add(f"blk.{l}.attn_v.weight", [HIDDEN, KVH * HD], Q6_K, s + 12)
        add(f"blk.{l}.attn_q_norm.weight", [HD], F32, s + 13, 0.2)
        add(f"blk.{l}.attn_k_norm.weight", [HD], F32, s + 14, 0.2)
        add(f"blk.{l}.attn_output.weight", [QH * HD, HIDDEN], Q4_K, s + 15)
        add(f"blk.{l}.ffn_gate.weight", [HIDDEN, FFN], Q4_K, s + 16)
        add(f"blk.{l}.ffn_up.weight", [HIDDEN, FFN], Q4_K, s + 17)
        add(f"blk.{l}.ffn_down.weight", [FFN, HIDDEN], Q6_K, s + 18)
        add(f"blk.{l}.ffn_gate_inp.scale", [HIDDEN], F32, s + 19, 0.5)
        add(f"blk.{l}.ffn_gate_inp.weight", [HIDDEN, EXPERTS], F16, s + 20, 0.5)
        add(f"blk.{l}.ffn_down_exps.scale", [EXPERTS], F32, s + 21, 0.5)
        add(f"blk.{l}.ffn_gate_up_exps.weight", [HIDDEN, 2 * EXPERT_WIDTH, EXPERTS], Q4_K, s + 22)
        add(f"blk.{l}.ffn_down_exps.weight", [EXPERT_WIDTH, HIDDEN, EXPERTS], Q8_0, s + 23)
        add(f"blk.{l}.layer_output_scale.weight", [1], F32, s + 24, 0.5)
    add("output_norm.weight", [HIDDEN], F32, 2, 0.2)
    add("output.weight", [HIDDEN, VOCAB], Q6_K, 3)
    return t, enc


class Model:
    """The tensor table of the written file and host reads of its vectors
    (tensor_vector / tensor_row, src/gemma4/metal.rs:796-808)."""

    def __init__(self, path):
        self.file = open(path, "rb")
        self.mapping = mmap.mmap(self.file.fileno(), 0, access=mmap.ACCESS_READ)
        self.bytes = np.frombuffer(self.mapping, np.uint8)
        self.table = {t.name: t for t in gguf_file.read_tensors(self.mapping)}

    def raw(self, name):
        t = self.table[name]
        return self.bytes[t.absolute_offset:t.absolute_offset + t.byte_len]

    def vector(self, name):
        t = self.table[name]
        raw = self.raw(name)
        return raw.view(np.float32).copy() if t.kind == F32 else raw.view(np.float16).astype(np.float32)

    def row(self, name, index):
        cols = self.table[name].dimensions[0]
        return self.vector(name)[index * cols:(index + 1) * cols].copy()

    def close(self):
        del self.bytes
        self.mapping.close()
        self.file.close()


class HipGraph:
    """The graph's calls on the raw C ABI (the MetalContext methods the
    Gemma 4 graph uses, and the expert cache)."""

    def __init__(self, lib, model, path):
        self.lib, self.m = lib, model
        self.ctx = ctypes.c_void_p()
        self.ok(lib.dmhip_context_new(0, ctypes.byref(self.ctx)))
        self.buf = ctypes.c_void_p()
        self.ok(lib.dmhip_map_read_only(self.ctx, model.bytes.ctypes.data, model.bytes.size, ctypes.byref(self.buf)))
        self.kv = []
        for sliding, _, _ in LAYERS:
            h = ctypes.c_void_p()
            self.ok(lib.dmhip_new_kv_layer(self.ctx, KVH * HD, MAX_CONTEXT, int(sliding), WINDOW, ctypes.byref(h)))
            self.kv.append(h)
        from diskmule_amd.hip import _Layout
        layouts = (_Layout * len(LAYERS))()
        for l in range(len(LAYERS)):
            gu, dn = model.table[f"blk.{l}.ffn_gate_up_exps.weight"], model.table[f"blk.{l}.ffn_down_exps.weight"]
            layouts[l] = _Layout(EXPERTS, gu.absolute_offset, gu.byte_len // EXPERTS, dn.absolute_offset,
                                 dn.byte_len // EXPERTS)
        self.fd = os.open(path, os.O_RDONLY)
        self.cache = ctypes.c_void_p()
        self.ok(lib.dmhip_expert_cache_new_file(self.ctx, self.fd, layouts, len(LAYERS), 2, ctypes.byref(self.cache)))
        self.calls = []

    def ok(self, status):
        assert status == 0, self.lib.dmhip_last_error()

    def rms_norm(self, x, weight):
        x = _f32(x)
        out = np.zeros_like(x)
        w = None if weight is None else _f32(weight)
        self.ok(self.lib.dmhip_rms_norm(self.ctx, x.ctypes.data_as(f32p), x.size,
                                        None if w is None else w.ctypes.data_as(f32p), 0 if w is None else w.size,
                                        EPS, out.ctypes.data_as(f32p), out.size))
        self.calls.append(("rms_norm", out, capi.rms_norm(x, w, EPS)))
        return out

    def matvec(self, name, x, expert=None):
        """Gemma4MetalWeights::matvec / expert_matvec (src/gemma4/metal.rs:855-923)."""
        t = self.m.table[name]
        cols, rows = t.dimensions[0], t.dimensions[1]
        off, length = t.absolute_offset, t.byte_len
        x = _f32(x)
        y = np.zeros(rows, np.float32)
        self.ok(self.lib.dmhip_matvec_mapped(self.ctx, t.kind, rows, cols, self.buf, off, length,
                                             x.ctypes.data_as(f32p), x.size, y.ctypes.data_as(f32p), y.size))
        self.calls.append(("matvec " + name, y, capi.matvec(t.kind, rows, cols, self.m.raw(name), x)))
        return y

    def rope(self, values, heads, pairs, position, theta):
        v = _f32(values).copy()
        want = capi.rope_neox(v, heads, HD, pairs, position, theta)
        self.ok(self.lib.dmhip_rope_neox_in_place(self.ctx, v.ctypes.data_as(f32p), v.size, heads, HD, pairs,
                                                  position, theta))
        self.calls.append(("rope", v, want))
        return v

    def append_kv(self, layer, position, key, value):
        k, v = _f32(key), _f32(value)
        self.ok(self.lib.dmhip_append_kv(self.ctx, self.kv[layer], position, k.ctypes.data_as(f32p), k.size,
                                         v.ctypes.data_as(f32p), v.size))

    def attention_cached(self, layer, query):
        q = _f32(query)
        out = np.zeros_like(q)
        self.ok(self.lib.dmhip_attention_cached(self.ctx, q.ctypes.data_as(f32p), q.size, self.kv[layer], QH, KVH,
                                                HD, out.ctypes.data_as(f32p), out.size))
        return out

    def add(self, a, b):
        a, b = _f32(a), _f32(b)
        out = np.zeros_like(a)
        self.ok(self.lib.dmhip_add(self.ctx, a.ctypes.data_as(f32p), a.size, b.ctypes.data_as(f32p), b.size,
                                   out.ctypes.data_as(f32p), out.size))
        self.calls.append(("add", out, (a + b).astype(np.float32)))
        return out

    def gelu_mul(self, gate, up):
        g, u = _f32(gate), _f32(up)
        out = np.zeros_like(g)
        self.ok(self.lib.dmhip_gelu_mul(self.ctx, g.ctypes.data_as(f32p), g.size, u.ctypes.data_as(f32p), u.size,
                                        out.ctypes.data_as(f32p), out.size))
        self.calls.append(("gelu_mul", out, capi.gelu_mul(g, u)))
        return out

    def top_k_softmax(self, logits, k):
        x = _f32(logits)
        idx = (ctypes.c_size_t * k)()
        p = np.zeros(k, np.float32)
        self.ok(self.lib.dmhip_top_k_softmax(self.ctx, x.ctypes.data_as(f32p), x.size, k, idx,
                                             p.ctypes.data_as(f32p)))
        return [(int(idx[i]), np.float32(p[i])) for i in range(k)]

    def softcap(self, x, cap):
        x = _f32(x)
        out = np.zeros_like(x)
        self.ok(self.lib.dmhip_softcap(self.ctx, x.ctypes.data_as(f32p), x.size, cap, out.ctypes.data_as(f32p),
                                       out.size))
        self.calls.append(("softcap", out, capi.softcap(x, cap)))
        return out

    def streamed_expert(self, layer, expert, x):
        """ExpertCache::with_expert -> Gemma4::streamed_expert
        (src/expert.rs:138-164, src/gemma4/metal.rs:972-1000)."""
        slot, gu, dn = ctypes.c_size_t(), ctypes.c_void_p(), ctypes.c_void_p()
        cancelled = ctypes.c_int(0)
        self.ok(self.lib.dmhip_expert_acquire(self.cache, layer, expert, ctypes.byref(cancelled), ctypes.byref(slot),
                                              ctypes.byref(gu), ctypes.byref(dn)))
        try:
            gut = self.m.table[f"blk.{layer}.ffn_gate_up_exps.weight"]
            dnt = self.m.table[f"blk.{layer}.ffn_down_exps.weight"]
            gu_len, dn_len = gut.byte_len // EXPERTS, dnt.byte_len // EXPERTS
            x = _f32(x)
            gate_up = np.zeros(2 * EXPERT_WIDTH, np.float32)
            self.ok(self.lib.dmhip_matvec_owned(self.ctx, gut.kind, 2 * EXPERT_WIDTH, HIDDEN, gu, 0, gu_len,
                                                x.ctypes.data_as(f32p), x.size, gate_up.ctypes.data_as(f32p),
                                                gate_up.size))
            raw_gu = self.m.raw(gut.name)[expert * gu_len:(expert + 1) * gu_len]
            self.calls.append(("expert gate_up", gate_up, capi.matvec(gut.kind, 2 * EXPERT_WIDTH, HIDDEN, raw_gu, x)))
            act = self.gelu_mul(gate_up[:EXPERT_WIDTH], gate_up[EXPERT_WIDTH:])
            out = np.zeros(HIDDEN, np.float32)
            self.ok(self.lib.dmhip_matvec_owned(self.ctx, dnt.kind, HIDDEN, EXPERT_WIDTH, dn, 0, dn_len,
                                                act.ctypes.data_as(f32p), act.size, out.ctypes.data_as(f32p),
                                                out.size))
            raw_dn = self.m.raw(dnt.name)[expert * dn_len:(expert + 1) * dn_len]
            self.calls.append(("expert down", out, capi.matvec(dnt.kind, HIDDEN, EXPERT_WIDTH, raw_dn, act)))
            return out
        finally:
            self.ok(self.lib.dmhip_expert_release(self.cache, layer, slot.value))

    def stats(self):
        from diskmule_amd.hip import _Stats
        s = _Stats()
        self.ok(self.lib.dmhip_expert_cache_stats_get(self.cache, ctypes.byref(s)))
        return {n: getattr(s, n) for n, _ in _Stats._fields_}

    def close(self):
        self.lib.dmhip_expert_cache_free(self.cache)
        os.close(self.fd)
        for h in self.kv:
            self.lib.dmhip_kv_layer_free(h)
        self.lib.dmhip_buffer_free(self.buf)
        self.lib.dmhip_context_free(self.ctx)


class OracleGraph:
    """The same step on the CPU oracle (src/gemma4/cpu.rs's arithmetic per
    operation), with ring-buffer KV caches and the reference's LRU."""

    def __init__(self, model):
        self.m = model
        self.keys = [np.zeros((min(WINDOW if s else MAX_CONTEXT, MAX_CONTEXT), KVH * HD), np.float32)
                     for s, _, _ in LAYERS]
        self.values = [np.zeros_like(k) for k in self.keys]
        self.position = [0] * len(LAYERS)
        t = model.table["blk.0.ffn_gate_up_exps.weight"]
        d = model.table["blk.0.ffn_down_exps.weight"]
        self.lru = capi.Lru([EXPERTS] * len(LAYERS), 2, t.byte_len // EXPERTS, d.byte_len // EXPERTS)

    def rms_norm(self, x, weight):
        return capi.rms_norm(_f32(x), None if weight is None else _f32(weight), EPS)

    def matvec(self, name, x):
        t = self.m.table[name]
        return capi.matvec(t.kind, t.dimensions[1], t.dimensions[0], self.m.raw(name), _f32(x))

    def rope(self, values, heads, pairs, position, theta):
        return capi.rope_neox(_f32(values), heads, HD, pairs, position, theta)

    def append_kv(self, layer, position, key, value):
        cap = self.keys[layer].shape[0]
        self.keys[layer][position % cap] = key
        self.values[layer][position % cap] = value
        self.position[layer] = position + 1

    def attention_cached(self, layer, query):
        cap = self.keys[layer].shape[0]
        visible = min(self.position[layer], cap)
        return capi.attention(_f32(query), self.keys[layer], self.values[layer], cap, KVH * HD, QH, KVH, HD,
                              self.position[layer] - visible, visible)

    def add(self, a, b):
        return (_f32(a) + _f32(b)).astype(np.float32)

    def gelu_mul(self, gate, up):
        return capi.gelu_mul(_f32(gate), _f32(up))

    def top_k_softmax(self, logits, k):
        return [(e, np.float32(p)) for e, p in capi.top_k_softmax(_f32(logits), k)]

    def softcap(self, x, cap):
        return capi.softcap(_f32(x), cap)

    def streamed_expert(self, layer, expert, x):
        self.lru.acquire(layer, expert)
        gut, dnt = (self.m.table[f"blk.{layer}.ffn_gate_up_exps.weight"],
                    self.m.table[f"blk.{layer}.ffn_down_exps.weight"])
        gu_len, dn_len = gut.byte_len // EXPERTS, dnt.byte_len // EXPERTS
        raw_gu = self.m.raw(gut.name)[expert * gu_len:(expert + 1) * gu_len]
        raw_dn = self.m.raw(dnt.name)[expert * dn_len:(expert + 1) * dn_len]
        gate_up = capi.matvec(gut.kind, 2 * EXPERT_WIDTH, HIDDEN, raw_gu, _f32(x))
        act = capi.gelu_mul(gate_up[:EXPERT_WIDTH], gate_up[EXPERT_WIDTH:])
        return capi.matvec(dnt.kind, HIDDEN, EXPERT_WIDTH, raw_dn, act)


def decode_step(g, m, token, position, record):
    """forward_token_inner (src/gemma4/metal.rs:577-794) on graph `g`."""
    hidden = (m.row("token_embd.weight", token) * np.float32(math.sqrt(HIDDEN))).astype(np.float32)
    for l, (sliding, pairs, theta) in enumerate(LAYERS):
        p = f"blk.{l}."
        residual = hidden
        attn_in = g.rms_norm(residual, m.vector(p + "attn_norm.weight"))
        q = g.matvec(p + "attn_q.weight", attn_in)
        k = g.matvec(p + "attn_k.weight", attn_in)
        v = g.matvec(p + "attn_v.weight", attn_in)
        qn, kn = m.vector(p + "attn_q_norm.weight"), m.vector(p + "attn_k_norm.weight")
        q = np.concatenate([g.rms_norm(q[h * HD:(h + 1) * HD], qn) for h in range(QH)])
        k = np.concatenate([g.rms_norm(k[h * HD:(h + 1) * HD], kn) for h in range(KVH)])
        v = np.concatenate([g.rms_norm(v[h * HD:(h + 1) * HD], None) for h in range(KVH)])
        q = g.rope(q, QH, pairs, position, theta)
        k = g.rope(k, KVH, pairs, position, theta)
        g.append_kv(l, position, k, v)
        att = g.attention_cached(l, q)
        record.setdefault("attention", []).append(att)
        proj = g.matvec(p + "attn_output.weight", att)
        proj = g.rms_norm(proj, m.vector(p + "post_attention_norm.weight"))
        attn_out = g.add(residual, proj)
        shared_in = g.rms_norm(attn_out, m.vector(p + "ffn_norm.weight"))
        gate = g.matvec(p + "ffn_gate.weight", shared_in)
        up = g.matvec(p + "ffn_up.weight", shared_in)
        shared = g.matvec(p + "ffn_down.weight", g.gelu_mul(gate, up))
        shared = g.rms_norm(shared, m.vector(p + "post_ffw_norm_1.weight"))
        routed_in = g.rms_norm(attn_out, m.vector(p + "pre_ffw_norm_2.weight"))
        router_in = g.rms_norm(attn_out, None)
        inv = np.float32(1.0) / np.float32(math.sqrt(HIDDEN))
        router_in = (router_in * (m.vector(p + "ffn_gate_inp.scale") * inv).astype(np.float32)).astype(np.float32)
        logits = g.matvec(p + "ffn_gate_inp.weight", router_in)
        selected = g.top_k_softmax(logits, USED)
        record.setdefault("selected", []).append([e for e, _ in selected])
        record.setdefault("router_logits", []).append(logits)
        down_scale = m.vector(p + "ffn_down_exps.scale")
        routed = np.zeros(HIDDEN, np.float32)
        for e, prob in selected:
            out = g.streamed_expert(l, e, routed_in)
            scale = np.float32(prob * down_scale[e])
            routed = np.array([fma32(a, scale, c) for a, c in zip(out, routed)], dtype=np.float32)
        routed = g.rms_norm(routed, m.vector(p + "post_ffw_norm_2.weight"))
        combined = g.add(shared, routed)
        combined = g.rms_norm(combined, m.vector(p + "post_ffw_norm.weight"))
        hidden = g.add(attn_out, combined)
        hidden = (hidden * m.vector(p + "layer_output_scale.weight")[0]).astype(np.float32)
        record.setdefault("hidden", []).append(hidden)
    normed = g.rms_norm(hidden, m.vector("output_norm.weight"))
    return g.softcap(g.matvec("output.weight", normed), SOFTCAP)


def test_gemma4_decode_step_through_the_c_abi(tmp_path):
    tensors, _ = _tensors()
    path = tmp_path / "gemma4-small.gguf"
    gguf_file.write(path, tensors)
    model = Model(path)
    lib = load_library()
    gpu = HipGraph(lib, model, str(path))
    cpu = OracleGraph(model)
    try:
        for position, token in enumerate(TOKENS):
            print(f"gemma4 step position={position} token={token}", flush=True)
            rec_g, rec_c = {}, {}
            got = decode_step(gpu, model, token, position, rec_g)
            want = decode_step(cpu, model, token, position, rec_c)
            # every library call against the oracle on the same inputs
            for name, out, ref in gpu.calls:
                if name == "add":
                    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), name
                elif name == "rms_norm" or name == "rope":
                    assert_close(out, ref, f"{name} at position {position}")
                else:
                    assert_close(out, ref, f"{name} at position {position}")
            gpu.calls.clear()
            # the independent composition of the whole step
            for l in range(len(LAYERS)):
                gap = np.sort(rec_c["router_logits"][l])[::-1]
                print(f"  layer {l}: experts gpu={rec_g['selected'][l]} cpu={rec_c['selected'][l]} "
                      f"gap {gap[USED - 1] - gap[USED]:.3g}", flush=True)
                assert rec_g["selected"][l] == rec_c["selected"][l]
                assert_close(rec_g["attention"][l], rec_c["attention"][l], f"attention layer {l}")
                assert_close(rec_g["hidden"][l], rec_c["hidden"][l], f"hidden layer {l}")
            e, c = assert_close(got, want, f"logits at position {position}")
            print(f"  logits rel_err={e:.2e} cosine={c:.9f} argmax gpu={int(np.argmax(got))} "
                  f"cpu={int(np.argmax(want))}", flush=True)
        # the file-backed cache made the reference's LRU decisions
        st, ref = gpu.stats(), cpu.lru.stats()
        for key in ("hits", "misses", "evictions", "reads", "bytes_read", "resident_bytes"):
            assert st[key] == ref[key], (key, st[key], ref[key])
        assert st["misses"] > 0 and st["evictions"] > 0 and st["hits"] + st["misses"] == 2 * USED * len(TOKENS)
        for h in gpu.kv:
            assert lib.dmhip_kv_layer_position(h) == len(TOKENS)
    finally:
        gpu.close()
        model.close()
