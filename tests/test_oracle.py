"""Pins the CPU oracle (oracle/dm_oracle.c) before anything is checked
against it: the reference's own known answers, an independent numpy
restatement, exact-rational brute force, and textbook routines."""
import numpy as np
import pytest

from diskmule_amd import synth
from oracle import capi, numpy_ref
from tests.exact import fma32, fold_dot

ERR = {"InvalidElementCount": capi.INVALID_ELEMENT_COUNT, "UnsupportedType": capi.UNSUPPORTED_TYPE,
       "InvalidVectorLength": capi.INVALID_VECTOR_LENGTH, "InvalidTopK": capi.INVALID_TOP_K}


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---- the reference's known answers (src/cpu.rs:670-833) ------------------

@pytest.mark.parametrize("name", ["f32_decode", "f16_decode", "q5_0_decode", "q8_0_decode",
                                  "q4_k_decode", "q6_k_decode"])
def test_decoder_known_answers(golden, name):
    kat, _ = golden
    case = kat[name]
    out = capi.dequantize(case["type"], case["encoded"], len(case["expected"]))
    assert np.array_equal(bits(out), bits(case["expected"]))


def test_q4_k_scale_min_known_answer(golden):
    case = golden[0]["q4_k_scale_min"]
    assert list(capi.scale_min_q4_k(case["index"], case["scales"])) == case["expected"]


def test_matvec_known_answer(golden):
    c = golden[0]["matvec_row_major"]
    out = capi.matvec(c["type"], c["rows"], c["columns"], c["encoded"], c["input"], threads=1)
    assert out.tolist() == c["expected"]


def test_rejects_bad_lengths_and_unsupported_types(golden):
    kat = golden[0]
    for name in ("reject_q4_k_element_count", "reject_q5_k_unsupported"):
        c = kat[name]
        status = capi.dequantize_status(c["type"], np.zeros(c["encoded_len"], np.uint8), c["elements"])
        assert status == ERR[c["expected_error"]]


def test_rms_norm_known_answer(golden):
    c = golden[0]["rms_norm"]
    assert np.array_equal(bits(capi.rms_norm(c["input"], None, c["epsilon"])), bits(c["expected_unweighted"]))
    assert np.array_equal(bits(capi.rms_norm(c["input"], c["weight"], c["epsilon"])), bits(c["expected_weighted"]))
    assert capi.rms_norm_status(c["input"], c["bad_weight"], c["epsilon"], 2) == ERR[c["expected_error"]]
    # epsilon must be finite and positive; empty input is rejected
    assert capi.rms_norm_status(c["input"], None, 0.0, 2) == capi.INVALID_POSITIVE_PARAMETER
    assert capi.rms_norm_status([], None, 1e-6, 0) == capi.EMPTY_INPUT


def test_softmax_top_k_argmax_known_answers(golden):
    kat = golden[0]
    c = kat["softmax_stable"]
    p = capi.softmax([float(v) for v in c["input"]])
    assert abs(float(p.sum()) - c["sum"]) < c["sum_tolerance"]
    assert p[-1] == c["expected_last"]
    c = kat["top_k"]
    assert [list(t) for t in capi.top_k_softmax(c["logits"], c["k"])] == c["expected"]
    assert capi.argmax(kat["argmax_ties"]["input"]) == kat["argmax_ties"]["expected"]
    c = kat["top_k_zero"]
    assert capi.top_k_softmax_status(c["logits"], c["k"]) == ERR[c["expected_error"]]


def test_expert_lru_known_answer(golden):
    c = golden[0]["expert_lru"]
    lay = c["layout"]
    lru = capi.Lru([lay["expert_count"]], c["slots_per_layer"], lay["gate_up_bytes"], lay["down_bytes"])
    for layer, expert, _, _ in c["accesses"]:
        lru.acquire(layer, expert)
    assert lru.stats() == c["expected_stats"]


# ---- textbook routines and the independent numpy restatement --------------

def test_f16_widening_matches_numpy_for_every_pattern():
    # Through the array path (dequantize F16), so no value passes through a
    # C double, which would quiet signalling NaNs.  src/cpu.rs:647-660 keeps
    # NaN payloads; numpy's float16 -> float32 does too.
    patterns = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = capi.dequantize(1, patterns.view(np.uint8), patterns.size)
    assert np.array_equal(bits(ours), bits(numpy_ref.f16_bits_to_f32(patterns)))
    # subnormals are frac * 2^-24 exactly
    sub = np.arange(1, 1024, dtype=np.uint16)
    assert np.array_equal(capi.dequantize(1, sub.view(np.uint8), sub.size),
                          (sub.astype(np.float64) * 2.0 ** -24).astype(np.float32))


@pytest.mark.parametrize("kind,seed", [(12, 1), (14, 2), (8, 3)])
def test_decoders_match_the_metal_indexed_numpy_restatement(kind, seed):
    rows, cols = 64, 1024
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(seed))
    # exercise the f16 edge cases in the block scales too
    block = synth.BLOCK[kind][1]
    blocks = w.reshape(-1, block).copy()
    d_off = 208 if kind == 14 else 0
    specials = [0x0001, 0x03FF, 0x8001, 0x7BFF, 0xFBFF, 0x0000, 0x8000, 0x7C00]
    for i, s in enumerate(specials):
        blocks[i, d_off:d_off + 2] = np.array([s], dtype="<u2").view(np.uint8)
    enc = blocks.reshape(-1)
    a = capi.dequantize(kind, enc, rows * cols)
    b = numpy_ref.dequantize(kind, enc)
    both_nan = np.isnan(a) & np.isnan(b)
    assert np.array_equal(bits(a)[~both_nan], bits(b)[~both_nan])


def test_q5_0_matches_numpy_restatement():
    rng = np.random.default_rng(5)
    enc = rng.integers(0, 256, size=22 * 40, dtype=np.uint8)
    enc.reshape(40, 22)[:, 0:2] = np.array([0x3400], dtype="<u2").view(np.uint8)
    assert np.array_equal(bits(capi.dequantize(6, enc, 40 * 32)), bits(numpy_ref.dequantize(6, enc)))


# ---- matvec: exact-rational brute force of the fma fold ---------------------

@pytest.mark.parametrize("kind,seed,cols", [(12, 11, 512), (14, 12, 512), (8, 13, 256)])
def test_matvec_equals_exact_sequential_fma_fold(kind, seed, cols):
    rows = 3
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(seed))
    x = synth.normal(synth.activation_seed(seed), cols)
    got = capi.matvec(kind, rows, cols, w, x, threads=2)
    deq = numpy_ref.dequantize(kind, w).reshape(rows, cols)
    want = np.array([fold_dot(deq[r], x) for r in range(rows)], dtype=np.float32)
    assert np.array_equal(bits(got), bits(want))
    # the check is sensitive to the fold order: a reversed fold differs
    rev = np.array([fold_dot(deq[r][::-1], x[::-1]) for r in range(rows)], dtype=np.float32)
    assert not np.array_equal(bits(rev), bits(want))


def test_matvec_bf16_equals_exact_fold():
    rows, cols = 4, 96
    w = synth.to_bf16_bits(synth.normal(77, rows * cols) * np.float32(0.02))
    x = synth.normal(78, cols)
    got = capi.matvec_bf16(rows, cols, w, x, threads=1)
    wf = synth.bf16_bits_to_f32(w).reshape(rows, cols)
    want = np.array([fold_dot(wf[r], x) for r in range(rows)], dtype=np.float32)
    assert np.array_equal(bits(got), bits(want))


def test_matvec_threads_do_not_change_bits():
    w = synth.quantized_matrix(12, 97, 512, synth.weight_seed(21))
    x = synth.normal(22, 512)
    a = capi.matvec(12, 97, 512, w, x, threads=1)
    b = capi.matvec(12, 97, 512, w, x, threads=7)
    assert np.array_equal(bits(a), bits(b))


def test_matvec_validation_order():
    x = np.zeros(256, np.float32)
    enc = np.zeros(144, np.uint8)
    assert capi.matvec_status(12, 1, 256, enc, x[:10], 1) == capi.INVALID_INPUT_LENGTH
    assert capi.matvec_status(12, 1, 256, enc, x, 2) == capi.INVALID_OUTPUT_LENGTH
    assert capi.matvec_status(12, 1, 100, enc, x[:100], 1) == capi.INVALID_ELEMENT_COUNT
    assert capi.matvec_status(12, 1, 256, enc[:100], x, 1) == capi.INVALID_BYTE_LENGTH
    assert capi.matvec_status(13, 1, 256, np.zeros(176, np.uint8), x, 1) == capi.UNSUPPORTED_TYPE
    assert capi.matvec_status(12, 0, 256, enc[:0], x, 0) == capi.OK


# ---- argmax / top-k against numpy's lexsort --------------------------------

def _np_top_k(logits, k):
    v = np.asarray(logits, dtype=np.float32)
    # total_cmp order: -0.0 < +0.0; ties by ascending index
    key = v.view(np.int32).astype(np.int64)
    key = np.where(key < 0, -(key & 0x7FFFFFFF) - 1, key)
    order = np.lexsort((np.arange(v.size), -key))
    return order[:k]


def test_top_k_and_argmax_match_lexsort_with_ties_and_signed_zero():
    rng = np.random.default_rng(3)
    for trial in range(50):
        n = int(rng.integers(1, 300))
        v = rng.integers(-4, 5, size=n).astype(np.float32) * np.float32(0.5)
        v[rng.random(n) < 0.1] = -0.0
        k = int(rng.integers(1, n + 1))
        sel = capi.top_k_softmax(v, k)
        assert [s[0] for s in sel] == _np_top_k(v, k).tolist()
        assert capi.argmax(v) == int(_np_top_k(v, 1)[0])
    assert capi.argmax([-0.0, 0.0]) == 1
    assert capi.argmax_status([1.0, np.nan]) == capi.NON_FINITE
    assert capi.argmax_status([]) == capi.EMPTY_INPUT


def test_top_k_probabilities_are_a_softmax_of_the_selected_logits():
    v = synth.normal(31, 128)
    sel = capi.top_k_softmax(v, 8)
    ids = [s[0] for s in sel]
    chosen = v[ids].astype(np.float64)
    ref = np.exp(chosen - chosen.max())
    ref /= ref.sum()
    assert np.allclose([s[1] for s in sel], ref, rtol=1e-6, atol=1e-7)


# ---- compositions ----------------------------------------------------------

def test_dense_ffn_is_the_composition_of_its_parts():
    hidden, ffn, batch = 256, 512, 2
    g = synth.quantized_matrix(12, ffn, hidden, synth.weight_seed(3, 0))
    u = synth.quantized_matrix(12, ffn, hidden, synth.weight_seed(3, 1))
    d = synth.quantized_matrix(14, hidden, ffn, synth.weight_seed(3, 2))
    h = synth.normal(synth.activation_seed(3), batch * hidden).reshape(batch, hidden)
    out = capi.dense_ffn(batch, hidden, ffn, 12, g, 12, u, 14, d, h)
    for b in range(batch):
        n = capi.rms_norm(h[b], None, 1e-6)
        gv = capi.matvec(12, ffn, hidden, g, n)
        uv = capi.matvec(12, ffn, hidden, u, n)
        a = np.array([capi.silu(float(gi)) for gi in gv], dtype=np.float32) * uv
        want = capi.matvec(14, hidden, ffn, d, a)
        assert np.array_equal(bits(out[b]), bits(want))
    # silu: the two branches of the stable sigmoid agree with the closed form
    for v in (-30.0, -1.5, -0.0, 0.0, 0.75, 12.0):
        assert np.isclose(float(capi.silu(v)), v / (1.0 + np.exp(-v)), rtol=1e-6, atol=1e-12)


# ---- GLM expert activation (src/glm52/expert.rs:260-267) --------------------
#
# orc_silu_mul_glm evaluates (g / (1 + exp(-g))) * u in f32: one exp, then
# the sum, the quotient and the product each round once.  Against the exact
# value computed in float64 its relative error is at most the exp's (glibc
# expf: under 1 ulp; 2 allowed) plus three roundings of 2^-24, so 6 * 2^-24,
# with two subnormal quanta of absolute slack where the product underflows.
# Below g = -88.72 the f32 exp(-g) overflows to +inf and the quotient is -0,
# as the reference's f32 code computes it; the float64 check stops at -88.

GLM_REL = 6.0 * 2.0 ** -24
GLM_ABS = 2.0 * 2.0 ** -149


def _glm_activation_excess(got, gate, up) -> float:
    """Largest |got - exact| / bound over the elements (<= 1 passes)."""
    g = np.asarray(gate, dtype=np.float64)
    u = np.asarray(up, dtype=np.float64)
    exact = g / (1.0 + np.exp(-g)) * u
    err = np.abs(np.asarray(got, dtype=np.float64) - exact)
    return float((err / (GLM_REL * np.abs(exact) + GLM_ABS)).max())


def _glm_inputs(seed=61, count=12000):
    """Gates over [-88, 88] (uniform, plus a log-spread of small magnitudes
    of both signs) and ups of magnitude 1e-3 .. 1e3 of both signs."""
    rng = np.random.default_rng(seed)
    g = np.concatenate([rng.uniform(-88.0, 88.0, count // 2),
                        np.sign(rng.uniform(-1, 1, count // 2)) * 10.0 ** rng.uniform(-30, 1.9, count // 2)])
    u = rng.standard_normal(count) * 10.0 ** rng.uniform(-3, 3, count)
    return g.astype(np.float32), u.astype(np.float32)


def test_glm_expert_activation_against_float64():
    g, u = _glm_inputs()
    got = capi.silu_mul_glm(g, u)
    assert _glm_activation_excess(got, g, u) <= 1.0


def test_glm_expert_activation_checks_catch_planted_mistakes():
    """The float64 check rejects each plausible slip in a numpy f32
    restatement of the formula: exp(+g), 1 - exp(-g), the up factor dropped,
    the sigmoid without the gate factor, and g / exp(-g)."""
    g, u = _glm_inputs(62, 4000)
    gf, uf = g.astype(np.float32), u.astype(np.float32)
    one = np.float32(1.0)
    with np.errstate(over="ignore", divide="ignore", invalid="ignore"):
        right = (gf / (one + np.exp(-gf))) * uf
        slips = {
            "exp(+g)": (gf / (one + np.exp(gf))) * uf,
            "1 - exp(-g)": (gf / (one - np.exp(-gf))) * uf,
            "no up": gf / (one + np.exp(-gf)),
            "sigmoid only": (one / (one + np.exp(-gf))) * uf,
            "no one": (gf / np.exp(-gf)) * uf,
        }
        assert _glm_activation_excess(right, g, u) <= 1.0
        for name, wrong in slips.items():
            assert not _glm_activation_excess(wrong, g, u) <= 1.0, name


def test_glm_expert_activation_against_the_pinned_silu():
    """Against orc_silu (pinned on its two branches) times up: the two
    evaluation orders differ by a few roundings, never more."""
    g, u = _glm_inputs(63, 3000)
    keep = g >= -87.0  # orc_silu's exp(g) branch has no overflow; compare where both are finite
    g, u = g[keep], u[keep]
    got = capi.silu_mul_glm(g, u)
    via_silu = np.array([capi.silu(float(a)) for a in g], dtype=np.float32) * u
    rel = np.abs(got.astype(np.float64) - via_silu) / (np.abs(via_silu.astype(np.float64)) + GLM_ABS)
    assert float(rel.max()) <= 12.0 * 2.0 ** -24


def test_glm_expert_activation_special_values():
    """Exact results where the formula leaves no rounding: g = +-0 gives a
    signed zero; for g >= 17 the f32 exp(-g) is below half an ulp of 1, so the
    result is the single rounding of g * u; past g = -88.72 exp(-g) overflows
    and the result is -0 (times the sign of u); inf and NaN propagate as
    IEEE arithmetic says."""
    def one(gv, uv):
        return capi.silu_mul_glm(np.float32([gv]), np.float32([uv]))[0]

    assert bits(one(0.0, 1.0)) == 0 and bits(one(-0.0, 1.0)) == 0x80000000
    assert bits(one(0.0, -2.5)) == 0x80000000
    for gv in (17.0, 30.0, 88.0, 1e4):
        for uv in (1.0, 0.1, -3.7, 1e-20):
            want = np.float32(np.float32(gv) * np.float32(uv))
            assert bits(one(gv, uv)) == bits(want), (gv, uv)
    for gv in (-30.0, -60.0, -88.0):
        got = one(gv, 1.5)
        assert got < 0 and _glm_activation_excess([got], [gv], [1.5]) <= 1.0, gv
    assert bits(one(-89.0, 2.0)) == 0x80000000 and bits(one(-1e4, -2.0)) == 0
    assert one(float("inf"), 2.0) == float("inf") and one(float("inf"), -2.0) == float("-inf")
    assert np.isnan(one(float("nan"), 1.0)) and np.isnan(one(float("-inf"), 1.0))


def test_moe_layer_is_the_composition_of_its_parts():
    hidden, width, experts, k, batch = 256, 256, 16, 4, 3
    router = synth.to_bf16_bits(synth.normal(41, experts * hidden) * np.float32(0.02))
    gu_row, dn_row = synth.row_bytes(12, hidden), synth.row_bytes(14, width)
    gu = synth.quantized_matrix(12, experts * 2 * width, hidden, 42)
    dn = synth.quantized_matrix(14, experts * hidden, width, 43)
    x = synth.normal(44, batch * hidden).reshape(batch, hidden)
    sel, wts, out = capi.moe_layer(batch, hidden, width, experts, k, router, 12, gu, 14, dn, x)
    for t in range(batch):
        logits = capi.matvec_bf16(experts, hidden, router, x[t])
        top = capi.top_k_softmax(logits, k)
        assert [e for e, _ in top] == sel[t].tolist()
        acc = np.zeros(hidden, np.float32)
        for e, p in top:
            g_u = capi.matvec(12, 2 * width, hidden, gu[e * 2 * width * gu_row:(e + 1) * 2 * width * gu_row], x[t])
            act = capi.silu_mul_glm(g_u[:width], g_u[width:])
            eo = capi.matvec(14, hidden, width, dn[e * hidden * dn_row:(e + 1) * hidden * dn_row], act)
            acc = np.array([fma32(a, b, c) for a, b, c in zip(eo, [p] * hidden, acc)], dtype=np.float32)
        assert np.array_equal(bits(out[t]), bits(acc))


def test_gemm_tokenwise_is_one_matvec_per_token():
    m, n, k = 3, 40, 512
    a = synth.to_bf16_bits(synth.normal(51, m * k))
    w = synth.quantized_matrix(12, n, k, 52)
    c = capi.gemm_tokenwise(12, m, n, k, a, w)
    for r in range(m):
        want = capi.matvec(12, n, k, w, synth.bf16_bits_to_f32(a[r * k:(r + 1) * k]))
        assert np.array_equal(bits(c[r]), bits(want))


# ---- LRU against an independent Python model of src/expert.rs:166-229 -------

def test_lru_matches_python_model_on_random_traces():
    rng = np.random.default_rng(8)
    experts, slots = 12, 4
    lru = capi.Lru([experts, experts], slots, 10, 6)
    model = [[None] * slots for _ in range(2)]
    last = [[0] * slots for _ in range(2)]
    clock = [0, 0]
    hits = misses = evictions = 0
    for _ in range(400):
        layer = int(rng.integers(0, 2))
        e = int(rng.integers(0, experts))
        slot, hit, ev = lru.acquire(layer, e)
        clock[layer] += 1
        if e in model[layer]:
            s = model[layer].index(e)
            last[layer][s] = clock[layer]
            hits += 1
            assert hit and slot == s and ev is None
            continue
        misses += 1
        s = min(range(slots), key=lambda i: (model[layer][i] is not None, last[layer][i], i))
        want_ev = model[layer][s]
        if want_ev is not None:
            evictions += 1
        model[layer][s] = e
        last[layer][s] = clock[layer]
        assert (not hit) and slot == s and ev == want_ev
    st = lru.stats()
    assert (st["hits"], st["misses"], st["evictions"]) == (hits, misses, evictions)
    assert st["reads"] == 2 * misses and st["bytes_read"] == 16 * misses
    assert st["resident_bytes"] == 2 * slots * 16


def test_softcap_matches_float64_and_its_invariants():
    """src/cpu.rs:263-273 on the reference's fixture input (src/metal.rs:
    2166-2168, 2231-2235: ((i % 31) - 15) * 0.071, cap 30) and a wide range:
    within 2 ulp of cap * tanh(x / cap) in float64, odd, bounded by the cap,
    identity-like near zero; caps that are not finite and positive are
    rejected (InvalidPositiveParameter)."""
    fixture = np.array([((i % 31) - 15) * 0.071 for i in range(513)], dtype=np.float32)
    wide = np.concatenate([fixture, np.float32([0.0, -0.0, 1e-30, -1e-30, 29.9, -29.9, 30.0, 1e4, -1e4, 3.4e38,
                                                -3.4e38])])
    for cap in (30.0, 1.5, 50.0):
        got = capi.softcap(wide, cap)
        want = cap * np.tanh(wide.astype(np.float64) / cap)
        ulp = np.spacing(np.maximum(np.abs(want), 1e-38).astype(np.float32)).astype(np.float64)
        assert (np.abs(got - want) <= 2 * ulp).all(), cap
        assert (np.abs(got) <= cap).all()
        np.testing.assert_array_equal(capi.softcap(-wide, cap), -got)
    small = capi.softcap(np.float32([1e-6, -2e-7]), 30.0)
    np.testing.assert_allclose(small, [1e-6, -2e-7], rtol=1e-6)
    for cap in (0.0, -1.0, float("inf"), float("nan")):
        assert capi.softcap_status(fixture, cap) == 11

