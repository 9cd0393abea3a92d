"""GPU parity of decode attention over a KV ring (MetalContext::new_kv_layer,
append_kv, attention_cached, attention: src/metal.rs:1196-1511) through the C
ABI: the reference's own known answers, the oracle and float64 on the same
fp32 scores within the rounding budget of tests/tolerance.py, and the
reference's validation errors in its order."""
import numpy as np
import pytest

from diskmule_amd import HipError
from oracle import capi
from tests.tolerance import assert_attention_close, attention_budget, attention_exact

pytestmark = pytest.mark.gpu


def fill_layer(ctx, layer, keys, values):
    for p in range(keys.shape[0]):
        ctx.append_kv(layer, p, keys[p], values[p])


def expect_error(variant, fn, *args, **detail):
    with pytest.raises(HipError) as e:
        fn(*args)
    assert e.value.variant == variant, str(e.value)
    for k, v in detail.items():
        assert e.value.detail.get(k) == v, (k, e.value.detail)
    return e.value


# ---- the reference's known answers -----------------------------------------------

def test_grouped_attention_uses_the_matching_kv_head(ctx):
    # src/gemma4/cpu.rs:967-976 through MetalContext::attention
    out = np.zeros(8, dtype=np.float32)
    ctx.attention([1, 0, 1, 0, 0, 1, 0, 1], [1, 0, 0, 1], [2, 3, 5, 7], 4, 2, 2, None, out)
    assert out.tolist() == [2, 3, 2, 3, 5, 7, 5, 7]


def test_sliding_attention_ignores_values_outside_the_window(ctx):
    # src/gemma4/cpu.rs:978-985
    out = np.zeros(2, dtype=np.float32)
    ctx.attention([1, 0], [1, 0, 1, 0], [100, 100, 2, 4], 1, 1, 2, 1, out)
    assert out.tolist() == [2, 4]


def test_grouped_sliding_attention_matches_the_cpu_reference(ctx):
    # src/metal.rs:2499-2541, tolerance 2e-6 there
    query = np.array([1.0, -0.5, 0.25, 0.75, -0.5, 1.0, 0.6, -0.2], dtype=np.float32)
    keys = np.array([0.5, 0.1, -0.2, 0.8, 0.9, -0.4, 0.3, 0.7, -0.6, 0.2, 1.0, -0.5], dtype=np.float32)
    values = np.array([10.0, 20.0, 30.0, 40.0, 1.0, 2.0, 3.0, 4.0, -2.0, 0.5, 7.0, -3.0], dtype=np.float32)
    out = np.zeros(8, dtype=np.float32)
    ctx.attention(query, keys, values, 4, 2, 2, 2, out)
    want = capi.attention(query, keys, values, 3, 4, 4, 2, 2, 1, 2)
    assert np.abs(out - want).max() <= 2e-6


def test_resident_kv_cache_wraps_at_the_sliding_window(ctx):
    # src/metal.rs:2543-2570
    cache = ctx.new_kv_layer(2, 10, 2)
    assert cache.capacity() == 2
    assert cache.allocated_bytes() == 32
    ctx.append_kv(cache, 0, [1.0, 0.0], [100.0, 100.0])
    ctx.append_kv(cache, 1, [1.0, 0.0], [2.0, 4.0])
    ctx.append_kv(cache, 2, [1.0, 0.0], [6.0, 8.0])
    out = np.zeros(2, dtype=np.float32)
    ctx.attention_cached([1.0, 0.0], cache, 1, 1, 2, out)
    assert np.abs(out - [4.0, 6.0]).max() <= 1e-6
    assert cache.position() == 3
    cache.truncate(2)
    assert cache.position() == 2
    cache.clear()
    assert cache.position() == 0
    cache.free()


# ---- parity with the oracle and float64 -----------------------------------------------

CACHED = [
    # qh, kvh, hd, max_context, window, positions, scale
    (1, 1, 2, 16, None, 5, 1.0),
    (4, 2, 8, 64, 16, 40, 1.0),          # ring wrapped twice
    (3, 1, 5, 100, 33, 70, 1.0),         # group 3, head dimension not a multiple of 4
    (8, 2, 64, 300, None, 257, 0.125),   # one past a 256-position chunk
    (16, 8, 256, 2048, 1024, 1500, 0.0625),  # Gemma 4 sliding layer, wrapped
    (16, 2, 512, 4096, None, 3000, 0.044),   # Gemma 4 full layer
    (12, 1, 128, 600, None, 513, 0.09),  # 12 heads per KV head
    (32, 2, 64, 200, None, 130, 0.125),  # 16 heads per KV head: two head groups
    (4, 4, 1024, 400, None, 300, 0.03),  # four value dims per thread
    (2, 1, 130, 90, 64, 90, 0.09),       # head dimension 130
    (6, 3, 16, 50, None, 50, 3.0),       # nearly one-hot softmax
]


@pytest.mark.parametrize("qh,kvh,hd,max_context,window,positions,scale", CACHED)
def test_attention_cached_parity(ctx, qh, kvh, hd, max_context, window, positions, scale):
    print(f"attention_cached qh={qh} kvh={kvh} hd={hd} window={window} positions={positions}", flush=True)
    rng = np.random.default_rng(qh * 7919 + hd * 31 + positions)
    width = kvh * hd
    keys = rng.standard_normal((positions, width)).astype(np.float32)
    values = rng.standard_normal((positions, width)).astype(np.float32)
    q = (rng.standard_normal(qh * hd) * scale).astype(np.float32)
    layer = ctx.new_kv_layer(width, max_context, window)
    cap = layer.capacity()
    fill_layer(ctx, layer, keys, values)
    out = np.zeros(qh * hd, dtype=np.float32)
    ctx.attention_cached(q, layer, qh, kvh, hd, out)
    visible = min(positions, cap)
    start = positions - visible
    # the ring as the layer holds it: position p in slot p % cap
    ring_k = np.zeros((cap, width), dtype=np.float32)
    ring_v = np.zeros((cap, width), dtype=np.float32)
    for p in range(positions):
        ring_k[p % cap] = keys[p]
        ring_v[p % cap] = values[p]
    # the device ring holds exactly these bytes
    got_k = ctx.copy_to_host(layer.keys_ptr(), cap * width * 4, np.float32).reshape(cap, width)
    assert np.array_equal(got_k[:min(positions, cap)], ring_k[:min(positions, cap)])
    want = capi.attention(q, ring_k, ring_v, cap, width, qh, kvh, hd, start, visible)
    exact, w, w2, _ = attention_exact(q, ring_k, ring_v, cap, width, qh, kvh, hd, start, visible)
    assert_attention_close(out, exact, w, w2, visible, "gpu vs float64")
    budget = attention_budget(w, w2, visible) + attention_budget(w, w2, visible, sequential=True)
    assert (np.abs(out - want).reshape(budget.shape) <= budget).all(), "gpu vs oracle"
    layer.free()


def test_host_cache_attention_with_and_without_window(ctx):
    rng = np.random.default_rng(17)
    qh, kvh, hd, seq = 8, 4, 96, 700
    width = kvh * hd
    keys = rng.standard_normal((seq, width)).astype(np.float32)
    values = rng.standard_normal((seq, width)).astype(np.float32)
    q = (rng.standard_normal(qh * hd) * 0.1).astype(np.float32)
    for window in (None, 1, 64, 699, 700, 5000):
        out = np.zeros(qh * hd, dtype=np.float32)
        ctx.attention(q, keys, values, qh, kvh, hd, window, out)
        start = 0 if window is None else max(seq - window, 0)
        visible = seq - start
        exact, w, w2, _ = attention_exact(q, keys, values, seq, width, qh, kvh, hd, start, visible)
        assert_attention_close(out, exact, w, w2, visible, f"window {window}")


def test_long_context_full_layer(ctx):
    # Gemma 4 full-attention shape at 16K positions, through host caches
    rng = np.random.default_rng(23)
    qh, kvh, hd, seq = 16, 2, 512, 16384
    width = kvh * hd
    keys = rng.standard_normal((seq, width)).astype(np.float32)
    values = rng.standard_normal((seq, width)).astype(np.float32)
    q = (rng.standard_normal(qh * hd) * 0.044).astype(np.float32)
    out = np.zeros(qh * hd, dtype=np.float32)
    ctx.attention(q, keys, values, qh, kvh, hd, None, out)
    exact, w, w2, _ = attention_exact(q, keys, values, seq, width, qh, kvh, hd, 0, seq)
    assert_attention_close(out, exact, w, w2, seq, "16K positions")


def test_device_entry_points_match_the_host_ones(ctx):
    rng = np.random.default_rng(29)
    qh, kvh, hd, positions = 16, 8, 256, 300
    width = kvh * hd
    keys = rng.standard_normal((positions, width)).astype(np.float32)
    values = rng.standard_normal((positions, width)).astype(np.float32)
    q = (rng.standard_normal(qh * hd) * 0.0625).astype(np.float32)
    host_layer = ctx.new_kv_layer(width, 1024, 256)
    dev_layer = ctx.new_kv_layer(width, 1024, 256)
    kbuf, vbuf = ctx.device_array(keys), ctx.device_array(values)
    kp, vp = kbuf.device_ptr, vbuf.device_ptr
    for p in range(positions):
        ctx.append_kv(host_layer, p, keys[p], values[p])
        ctx.append_kv_device(dev_layer, p, kp + p * width * 4, width, vp + p * width * 4, width)
    assert dev_layer.position() == positions
    qbuf = ctx.device_array(q)
    obuf = ctx.new_owned_buffer(qh * hd * 4)
    ctx.attention_cached_device(qbuf.device_ptr, qh * hd, dev_layer, qh, kvh, hd, obuf.device_ptr, qh * hd)
    ctx.attention_result()
    got = obuf.read(0, qh * hd * 4, np.float32)
    want = np.zeros(qh * hd, dtype=np.float32)
    ctx.attention_cached(q, host_layer, qh, kvh, hd, want)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for b in (kbuf, vbuf, qbuf, obuf, host_layer, dev_layer):
        b.free()


def test_repeated_calls_are_deterministic(ctx):
    rng = np.random.default_rng(31)
    qh, kvh, hd, seq = 16, 2, 512, 5000
    width = kvh * hd
    keys = rng.standard_normal(seq * width).astype(np.float32)
    values = rng.standard_normal(seq * width).astype(np.float32)
    q = (rng.standard_normal(qh * hd) * 0.044).astype(np.float32)
    first = np.zeros(qh * hd, dtype=np.float32)
    ctx.attention(q, keys, values, qh, kvh, hd, None, first)
    for _ in range(3):
        again = np.zeros(qh * hd, dtype=np.float32)
        ctx.attention(q, keys, values, qh, kvh, hd, None, again)
        assert np.array_equal(again.view(np.uint32), first.view(np.uint32))


def test_many_chunks_combined_in_splits(ctx):
    # 16 query heads on one KV head at 70,000 positions: 547 chunks of 128,
    # combined in 18 splits that publish their sums, the last of which adds
    # them in split order
    print("split combine: qh=16 kvh=1 hd=64 positions=70000", flush=True)
    rng = np.random.default_rng(37)
    qh, kvh, hd, seq = 16, 1, 64, 70000
    width = kvh * hd
    keys = rng.standard_normal((seq, width)).astype(np.float32)
    values = rng.standard_normal((seq, width)).astype(np.float32)
    q = (rng.standard_normal(qh * hd) * 0.125).astype(np.float32)
    out = np.zeros(qh * hd, dtype=np.float32)
    ctx.attention(q, keys, values, qh, kvh, hd, None, out)
    exact, w, w2, _ = attention_exact(q, keys, values, seq, width, qh, kvh, hd, 0, seq)
    assert_attention_close(out, exact, w, w2, seq, "split combine")
    again = np.zeros(qh * hd, dtype=np.float32)
    ctx.attention(q, keys, values, qh, kvh, hd, None, again)
    assert np.array_equal(again.view(np.uint32), out.view(np.uint32))


# ---- non-finite scores ---------------------------------------------------------------

def test_non_finite_scores_are_rejected(ctx):
    k = np.ones(8, dtype=np.float32)
    out = np.zeros(2, dtype=np.float32)
    for q in ([np.nan, 0.0], [np.inf, 0.0], [-np.inf, 0.0]):
        expect_error("NonFinite", ctx.attention, q, k, k, 1, 1, 2, None, out, operation="softmax")
    # a clean call after a failed one succeeds (the flag belongs to one call)
    ctx.attention([1.0, 0.0], k, k, 1, 1, 2, None, out)
    assert out.tolist() == [1.0, 1.0]
    layer = ctx.new_kv_layer(2, 4, None)
    ctx.append_kv(layer, 0, [1.0, 0.0], [3.0, 4.0])
    qb = ctx.device_array(np.array([np.nan, 0.0], dtype=np.float32))
    ob = ctx.new_owned_buffer(8)
    ctx.attention_cached_device(qb.device_ptr, 2, layer, 1, 1, 2, ob.device_ptr, 2)
    expect_error("NonFinite", ctx.attention_result)
    with pytest.raises(HipError):
        ctx.attention_result()  # nothing pending
    # one result covers every device call since the previous one: a NaN in
    # the first of two calls is still reported after a clean second call
    good = ctx.device_array(np.array([1.0, 0.0], dtype=np.float32))
    ctx.attention_cached_device(qb.device_ptr, 2, layer, 1, 1, 2, ob.device_ptr, 2)
    ctx.attention_cached_device(good.device_ptr, 2, layer, 1, 1, 2, ob.device_ptr, 2)
    expect_error("NonFinite", ctx.attention_result)
    ctx.attention_cached_device(good.device_ptr, 2, layer, 1, 1, 2, ob.device_ptr, 2)
    ctx.attention_result()  # a new period starts clean
    # a host-slice call ends an open period and reports its device calls: a
    # NaN met by a pending device call makes the clean host call fail, and no
    # result is left to read afterwards
    host_out = np.zeros(2, dtype=np.float32)
    ctx.attention_cached_device(qb.device_ptr, 2, layer, 1, 1, 2, ob.device_ptr, 2)
    expect_error("NonFinite", ctx.attention_cached, [1.0, 0.0], layer, 1, 1, 2, host_out, operation="softmax")
    assert host_out.tolist() == [3.0, 4.0]  # the host call's own output is written
    with pytest.raises(HipError):
        ctx.attention_result()
    ctx.attention_cached_device(good.device_ptr, 2, layer, 1, 1, 2, ob.device_ptr, 2)
    ctx.attention_cached([1.0, 0.0], layer, 1, 1, 2, host_out)  # clean device call, clean host call
    ctx.attention_cached([1.0, 0.0], layer, 1, 1, 2, host_out)  # and a host call with nothing pending
    for b in (qb, ob, good, layer):
        b.free()


# ---- validation, in src/metal.rs's order ---------------------------------------------

def test_new_kv_layer_checks(ctx):
    e = expect_error("InvalidAttentionShape", ctx.new_kv_layer, 0, 10, None)
    assert e.detail == {"reason": "KV width and capacity must be non-zero"}
    expect_error("InvalidAttentionShape", ctx.new_kv_layer, 4, 0, None)
    expect_error("InvalidAttentionShape", ctx.new_kv_layer, 4, 10, 0)
    expect_error("Overflow", ctx.new_kv_layer, 2 ** 62, 8, None)
    layer = ctx.new_kv_layer(4, 10, 100)  # window past the context: capacity 10
    assert layer.capacity() == 10 and layer.allocated_bytes() == 320 and layer.position() == 0
    layer.free()


def test_append_kv_checks(ctx):
    layer = ctx.new_kv_layer(2, 2, None)
    expect_error("KvPosition", ctx.append_kv, layer, 1, [1, 0], [1, 0], expected=1, actual=0)
    expect_error("KvWidth", ctx.append_kv, layer, 0, [1, 0, 0], [1, 0], expected=2, actual=2)
    expect_error("KvWidth", ctx.append_kv, layer, 0, [1], [1, 0, 0], expected=2, actual=1)
    assert layer.position() == 0  # a failed append leaves the layer alone
    ctx.append_kv(layer, 0, [1, 0], [1, 0])
    ctx.append_kv(layer, 1, [1, 0], [1, 0])
    expect_error("KvContext", ctx.append_kv, layer, 2, [1, 0], [1, 0], position=2, limit=2)
    layer.truncate(5)
    assert layer.position() == 2  # truncate never moves forward
    layer.free()


def test_attention_cached_checks(ctx):
    layer = ctx.new_kv_layer(4, 8, None)
    out = np.zeros(4, dtype=np.float32)
    heads = "query heads must be a non-zero multiple of KV heads"
    lengths = "query and output must match query_heads * head_dimension"
    e = expect_error("InvalidAttentionShape", ctx.attention_cached, np.zeros(4), layer, 0, 1, 4, out)
    assert e.detail["reason"] == heads
    expect_error("InvalidAttentionShape", ctx.attention_cached, np.zeros(4), layer, 3, 2, 2, out)
    expect_error("Overflow", ctx.attention_cached, np.zeros(4), layer, 2, 1, 2 ** 63, out)
    e = expect_error("InvalidAttentionShape", ctx.attention_cached, np.zeros(3), layer, 2, 1, 2, out)
    assert e.detail["reason"] == lengths
    expect_error("InvalidAttentionShape", ctx.attention_cached, np.zeros(4), layer, 2, 1, 2, np.zeros(3, np.float32))
    expect_error("KvWidth", ctx.attention_cached, np.zeros(2), layer, 1, 1, 2, np.zeros(2, np.float32),
                 expected=2, actual=4)
    expect_error("EmptyInput", ctx.attention_cached, np.zeros(8), layer, 2, 1, 4, np.zeros(8, np.float32),
                 operation="attention")
    layer.free()


def test_attention_checks(ctx):
    out = np.zeros(4, dtype=np.float32)
    e = expect_error("InvalidAttentionShape", ctx.attention, np.zeros(4), np.zeros(4), np.zeros(4), 2, 0, 2,
                     None, out)
    assert e.detail["reason"] == "query heads must be a non-zero multiple of KV heads"
    shape = "key/value caches must have equal whole-position lengths"
    e = expect_error("InvalidAttentionShape", ctx.attention, np.zeros(4), np.zeros(4), np.zeros(6), 2, 1, 2,
                     None, out)
    assert e.detail["reason"] == shape
    expect_error("InvalidAttentionShape", ctx.attention, np.zeros(4), np.zeros(5), np.zeros(5), 2, 1, 2, None, out)
    expect_error("InvalidAttentionShape", ctx.attention, np.zeros(0), np.zeros(0), np.zeros(0), 2, 1, 0, None,
                 np.zeros(0, np.float32))
    expect_error("EmptyInput", ctx.attention, np.zeros(4), np.zeros(0), np.zeros(0), 2, 1, 2, None, out,
                 operation="attention")
    expect_error("EmptyInput", ctx.attention, np.zeros(4), np.zeros(4), np.zeros(4), 2, 1, 2, 0, out,
                 operation="attention window")
