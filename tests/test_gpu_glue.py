"""GPU parity of the Gemma 4 / GLM glue operators through the C ABI:
MetalContext::add, gelu_mul, softmax and rope_neox_in_place
(src/metal.rs:404-598), against the oracle (src/cpu.rs:144-225) on the
reference's own fixtures (src/metal.rs:2153-2229, with the reference's
tolerances) and on larger seeded inputs with derived bounds; the checks and
their order as src/metal.rs makes them."""
import numpy as np
import pytest

from diskmule_amd import HipError
from oracle import capi

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def expect_error(variant, fn, *args, **detail):
    with pytest.raises(HipError) as e:
        fn(*args)
    assert e.value.variant == variant, str(e.value)
    for k, v in detail.items():
        assert e.value.detail.get(k) == v, (k, e.value.detail)


FIXTURE = np.array([((i % 31) - 15.0) * 0.071 for i in range(513)], dtype=np.float32)


# ---- add ---------------------------------------------------------------------------

def test_add_known_answer_and_exactness(ctx):
    # src/metal.rs:2153-2161
    out = np.zeros(5, np.float32)
    ctx.add([1.0, 2.0, -3.0, 4.5, 0.25], [5.0, -2.0, 1.0, 0.5, 0.75], out)
    assert out.tolist() == [6.0, 0.0, -2.0, 5.0, 1.0]
    rng = np.random.default_rng(1)
    a = rng.standard_normal(1_000_003).astype(np.float32)
    b = (rng.standard_normal(a.size) * 1e3).astype(np.float32)
    out = np.zeros_like(a)
    ctx.add(a, b, out)
    assert np.array_equal(out.view(np.uint32), (a + b).view(np.uint32))  # one IEEE rounding each


def test_add_device_in_place(ctx):
    # the device form may write over either input
    rng = np.random.default_rng(4)
    a = rng.standard_normal(70_000).astype(np.float32)
    b = rng.standard_normal(a.size).astype(np.float32)
    da, db = ctx.device_array(a), ctx.device_array(b)
    ctx.add_device(a.size, da.device_ptr, db.device_ptr, da.device_ptr)
    ctx.add_device(a.size, da.device_ptr, db.device_ptr, db.device_ptr)
    assert np.array_equal(da.read(0, a.nbytes, np.float32), a + b)
    assert np.array_equal(db.read(0, a.nbytes, np.float32), (a + b) + b)
    ctx.add_device(0, 0, 0, 0)  # nothing to add
    for x in (da, db):
        x.free()


def test_add_checks(ctx):
    out = np.zeros(3, np.float32)
    expect_error("VectorLength", ctx.add, [1.0, 2.0], [1.0, 2.0, 3.0], out, left=2, right=3, output=3)
    expect_error("VectorLength", ctx.add, [1.0, 2.0], [1.0, 2.0], out, left=2, right=2, output=3)
    ctx.add([], [], np.zeros(0, np.float32))  # empty: nothing to do


# ---- gelu_mul ----------------------------------------------------------------------

def test_gelu_mul_reference_fixtures(ctx):
    # src/metal.rs:2195-2219 (tolerances 2e-6 and 2e-5 there)
    gate = FIXTURE[:67]
    up = (np.float32(1.25) - gate * np.float32(0.2)).astype(np.float32)
    out = np.zeros_like(gate)
    ctx.gelu_mul(gate, up, out)
    assert np.abs(out - capi.gelu_mul(gate, up)).max() <= 2e-6
    big_g = np.array([-80.0, -51.0, 37.0, 66.0, 90.0], np.float32)
    big_u = np.array([2.0, -3.0, 4.0, -5.0, 6.0], np.float32)
    out = np.zeros(5, np.float32)
    ctx.gelu_mul(big_g, big_u, out)
    assert np.abs(out - capi.gelu_mul(big_g, big_u)).max() <= 2e-5


def test_gelu_mul_random_and_device_form(ctx):
    rng = np.random.default_rng(2)
    gate = (rng.standard_normal(300_001) * 4).astype(np.float32)
    up = rng.standard_normal(gate.size).astype(np.float32)
    out = np.zeros_like(gate)
    ctx.gelu_mul(gate, up, out)
    want = capi.gelu_mul(gate, up).astype(np.float64)
    # the two tanhf differ by a few ulp: bound relative to the terms' sizes
    bound = 16 * U * (np.abs(gate) + np.abs(want / np.where(up == 0, 1, up))) * np.abs(up) + 1e-37
    assert (np.abs(out - want) <= bound).all()
    g, u, o = ctx.device_array(gate), ctx.device_array(up), ctx.new_owned_buffer(gate.nbytes)
    ctx.gelu_mul_device(gate.size, g.device_ptr, u.device_ptr, o.device_ptr)
    assert np.array_equal(o.read(0, gate.nbytes, np.float32), out)
    # in place: the output may be either input
    ctx.gelu_mul_device(gate.size, g.device_ptr, u.device_ptr, g.device_ptr)
    assert np.array_equal(g.read(0, gate.nbytes, np.float32), out)
    g.write(0, gate)
    ctx.gelu_mul_device(gate.size, g.device_ptr, u.device_ptr, u.device_ptr)
    assert np.array_equal(u.read(0, gate.nbytes, np.float32), out)
    # silu_mul's device form, in place over the gate
    u.write(0, up)
    want_silu = np.zeros_like(gate)
    ctx.silu_mul(gate, up, want_silu)
    ctx.silu_mul_device(gate.size, g.device_ptr, u.device_ptr, g.device_ptr)
    assert np.array_equal(g.read(0, gate.nbytes, np.float32), want_silu)
    for b in (g, u, o):
        b.free()


def test_gelu_mul_checks(ctx):
    out = np.zeros(2, np.float32)
    expect_error("EmptyInput", ctx.gelu_mul, [], [], np.zeros(0, np.float32), operation="GELU multiply")
    expect_error("InvalidVectorLength", ctx.gelu_mul, [1.0, 2.0], [1.0], out, operation="GELU multiply",
                 argument="up", expected=2, actual=1)
    expect_error("InvalidVectorLength", ctx.gelu_mul, [1.0, 2.0], [1.0, 2.0], np.zeros(3, np.float32),
                 argument="output", expected=2, actual=3)


# ---- softmax -----------------------------------------------------------------------

def test_softmax_reference_fixture(ctx):
    # src/metal.rs:2225-2229 (tolerance 2e-7 there)
    out = np.zeros_like(FIXTURE)
    ctx.softmax(FIXTURE, out)
    assert np.abs(out - capi.softmax(FIXTURE)).max() <= 2e-7


@pytest.mark.parametrize("n,scale", [(1, 1.0), (1000, 5.0), (262_144, 3.0), (70_001, 40.0)])
def test_softmax_against_float64(ctx, n, scale):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    out = np.zeros_like(x)
    ctx.softmax(x, out)
    e = np.exp(x.astype(np.float64) - x.max())
    want = e / e.sum()
    # exp of an exact difference (a few ulp each), a sum of n terms and one
    # division: relative error within (n + 8) u of each value's own size;
    # values below the smallest normal (2^-126) may be flushed to zero, as
    # the reference's Metal kernel flushes them
    assert (np.abs(out - want) <= (n + 8) * U * want + 2.0 ** -126).all()
    assert abs(out.astype(np.float64).sum() - 1.0) <= (n + 8) * U
    assert np.argmax(out) == np.argmax(x)


def test_softmax_checks(ctx):
    out = np.zeros(2, np.float32)
    expect_error("EmptyInput", ctx.softmax, [], np.zeros(0, np.float32), operation="softmax")
    expect_error("InvalidVectorLength", ctx.softmax, [1.0, 2.0], np.zeros(3, np.float32), operation="softmax",
                 argument="output", expected=2, actual=3)
    for bad in (np.nan, np.inf, -np.inf):
        expect_error("NonFinite", ctx.softmax, [1.0, bad], out, operation="softmax")


# ---- NeoX RoPE ---------------------------------------------------------------------

def test_rope_reference_fixture(ctx):
    # src/metal.rs:2181-2188 (tolerance 2e-5 there)
    v = np.array([(i - 24.0) * 0.125 for i in range(48)], dtype=np.float32)
    got = v.copy()
    ctx.rope_neox_in_place(got, 3, 16, 6, 37, 10_000.0)
    assert np.abs(got - capi.rope_neox(v, 3, 16, 6, 37, 10_000.0)).max() <= 2e-5


@pytest.mark.parametrize("heads,hd,pairs,position,theta", [(16, 256, 128, 4095, 10_000.0),
                                                           (2, 512, 64, 131_071, 1_000_000.0),
                                                           (8, 128, 64, 1, 10_000.0), (1, 2, 1, 7, 2.0)])
def test_rope_against_the_oracle(ctx, heads, hd, pairs, position, theta):
    print(f"rope heads={heads} hd={hd} pairs={pairs} position={position}", flush=True)
    rng = np.random.default_rng(hd + pairs)
    v = rng.standard_normal(heads * hd).astype(np.float32)
    got = v.copy()
    ctx.rope_neox_in_place(got, heads, hd, pairs, position, theta)
    want = capi.rope_neox(v, heads, hd, pairs, position, theta).astype(np.float64)
    # GPU powf / sinf / cosf against the C library's: each within a few ulp,
    # so the angle within a few ulp of itself; every output moves by at most
    # (|a| + |b|) times that, plus its own roundings
    half = hd // 2
    x = np.abs(v.reshape(heads, hd)).astype(np.float64)
    mag = np.concatenate([x[:, :half] + x[:, half:]] * 2, axis=1)
    ang = np.array([position * float(theta) ** float(np.float32(-2.0 * p) / np.float32(hd)) for p in range(half)])
    ang = np.concatenate([ang, ang])
    bound = mag * (8 * U * np.maximum(ang, 1.0) + 16 * U)
    assert (np.abs(got.reshape(heads, hd) - want.reshape(heads, hd)) <= bound).all()
    # dimensions past the rotated pairs are untouched, bit for bit
    g = got.reshape(heads, hd)
    assert np.array_equal(g[:, pairs:half], v.reshape(heads, hd)[:, pairs:half])
    # the device form writes the same bits
    d = ctx.device_array(v)
    ctx.rope_neox_device(d.device_ptr, v.size, heads, hd, pairs, position, theta)
    assert np.array_equal(d.read(0, v.nbytes, np.float32), got)
    d.free()


def test_rope_position_zero_is_the_identity(ctx):
    v = np.random.default_rng(3).standard_normal(4 * 64).astype(np.float32)
    got = v.copy()
    ctx.rope_neox_in_place(got, 4, 64, 32, 0, 10_000.0)
    assert np.array_equal(got, v)


def test_rope_checks_in_the_reference_order(ctx):
    v = np.zeros(8, np.float32)
    expect_error("InvalidRopeShape", ctx.rope_neox_in_place, v, 3, 4, 1, 0, 1.0, length=8, heads=3,
                 head_dimension=4)
    expect_error("InvalidRopeShape", ctx.rope_neox_in_place, v, 2 ** 62, 8, 1, 0, 1.0)
    expect_error("InvalidRopePairs", ctx.rope_neox_in_place, np.zeros(6, np.float32), 2, 3, 1, 0, 1.0)
    expect_error("InvalidRopePairs", ctx.rope_neox_in_place, v, 2, 4, 3, 0, 1.0)
    expect_error("InvalidPositiveParameter", ctx.rope_neox_in_place, v, 2, 4, 1, 0, 0.0,
                 operation="NeoX RoPE theta")
    expect_error("InvalidPositiveParameter", ctx.rope_neox_in_place, v, 2, 4, 1, 0, float("inf"))
    ones = np.ones(8, np.float32)
    ctx.rope_neox_in_place(ones, 2, 4, 0, 5, 1.0)  # no pairs: a no-op
    assert np.array_equal(ones, np.ones(8, np.float32))
    expect_error("VectorTooLarge", ctx.rope_neox_in_place, v, 2, 4, 1, 2 ** 32, 1.0)
