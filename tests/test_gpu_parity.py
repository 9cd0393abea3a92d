"""GPU parity: the HIP path through the C ABI against the CPU oracle on the
same seeded inputs.  Bit-exact for dequantized values, argmax and expert
ids; the north star's tolerance (tests/tolerance.py) for dot products."""
import numpy as np
import pytest

from diskmule_amd import ExpertCache, ExpertLayerLayout, HipError, synth
from diskmule_amd.hip import PinnedHostBuffer
from oracle import capi
from tests.tolerance import (CHANNEL_TOL_GEMM, CHANNEL_TOL_GEMV, assert_channel_close, assert_close,
                             assert_metal_tolerance, channel_err, exact_products, top2_gap)

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0, Q5_0, F16, F32 = 12, 14, 8, 6, 1, 0


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def dev(ctx, arr):
    return ctx.device_array(np.ascontiguousarray(arr))


def dev_out(ctx, nbytes):
    return ctx.new_owned_buffer(nbytes)


def test_device_is_gfx950(ctx):
    name = ctx.device_name()
    print("device:", name, flush=True)
    assert "gfx950" in name


# ---- dequantization: bit-exact ---------------------------------------------

@pytest.mark.parametrize("kind,rows,cols", [(Q4_K, 64, 4096), (Q6_K, 64, 4096), (Q8_0, 64, 4096),
                                            (Q6_K, 5, 768)])
def test_dequantize_is_bit_exact(ctx, kind, rows, cols):
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(kind))
    blocks = w.reshape(-1, synth.BLOCK[kind][1]).copy()
    d_off = 208 if kind == Q6_K else 0
    for i, s in enumerate([0x0001, 0x03FF, 0x8001, 0x7C00, 0xFC00, 0x7E01, 0x7C01, 0x0000, 0x8000]):
        blocks[i, d_off:d_off + 2] = np.array([s], dtype="<u2").view(np.uint8)
    enc = blocks.reshape(-1)
    buf = ctx.map_read_only(enc)
    got = ctx.dequantize(kind, buf, 0, enc.size, rows * cols)
    want = capi.dequantize(kind, enc, rows * cols)
    assert np.array_equal(bits(got), bits(want))


def test_dequantize_known_answers(ctx, golden):
    kat, _ = golden
    for name in ("f32_decode", "f16_decode", "q5_0_decode", "q8_0_decode", "q4_k_decode", "q6_k_decode"):
        c = kat[name]
        enc = np.array(c["encoded"], dtype=np.uint8)
        buf = ctx.map_read_only(enc)
        got = ctx.dequantize(c["type"], buf, 0, enc.size, len(c["expected"]))
        assert np.array_equal(bits(got), bits(c["expected"])), name


def test_dequantize_validation(ctx):
    buf = ctx.map_read_only(np.zeros(144, np.uint8))
    with pytest.raises(HipError) as e:
        ctx.dequantize(Q4_K, buf, 0, 144, 32)
    assert e.value.variant == "InvalidElementCount"
    with pytest.raises(HipError) as e:
        ctx.dequantize(13, buf, 0, 0, 0)
    assert e.value.variant == "UnsupportedTensorType"


# ---- matvec: the reference's Metal fixture (src/metal.rs:2256-2279) -------

def _metal_fixture(kind, rows):
    from tests.golden.make_golden import metal_matvec_fixture, metal_fixture_input
    cols, enc = metal_matvec_fixture(kind, rows)
    return cols, enc, metal_fixture_input(cols)


@pytest.mark.parametrize("kind", [F32, F16, Q5_0, Q8_0, Q4_K, Q6_K])
def test_encoded_matvec_kernels_match_the_cpu_reference(ctx, kind):
    rows = 3
    cols, enc, x = _metal_fixture(kind, rows)
    want = capi.matvec(kind, rows, cols, enc, x)
    got = np.zeros(rows, np.float32)
    ctx.matvec(kind, rows, cols, enc, x, got)
    assert_metal_tolerance(got, want, f"type {kind}")


@pytest.mark.parametrize("kind", [F32, F16, Q5_0])
@pytest.mark.parametrize("rows,cols,batch", [(4096, 4096, 1), (12288, 4096, 2), (1000, 2560, 3), (37, 544, 5),
                                             (70001, 256, 1), (9, 8192, 4), (300, 64, 2)])
def test_dense_gemv_matches_oracle(ctx, kind, rows, cols, batch):
    """F32 / F16 / Q5_0 rows on the wide-load GEMV: columns that are not a
    multiple of a 64-lane pass, odd row counts, 1-5 tokens (groups of up to
    4); Q5_0 blocks 2 bytes off a dword boundary in every other block (544
    columns, not whole block pairs, take the exact kernel)."""
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(160, kind))
    x = synth.normal(synth.activation_seed(160, cols), batch * cols).reshape(batch, cols)
    wb, xb, yb = dev(ctx, w), dev(ctx, x), dev_out(ctx, batch * rows * 4)
    ctx.matvec_device(kind, rows, cols, wb.device_ptr, batch, xb.device_ptr, yb.device_ptr)
    got = yb.read(0, batch * rows * 4, np.float32).reshape(batch, rows)
    for b in range(batch):
        assert_close(got[b], capi.matvec(kind, rows, cols, w, x[b]), f"type {kind} {rows}x{cols} token {b}")


def test_mapped_matvec_reads_a_nonzero_file_offset(ctx, golden):
    c = golden[0]["matvec_row_major"]
    enc = np.array(c["encoded"], dtype=np.uint8)
    mapping = ctx.map_read_only(np.concatenate([np.zeros(32, np.uint8), enc]))
    out = np.zeros(2, np.float32)
    ctx.matvec_mapped(F32, 2, 2, mapping, 32, enc.size, c["input"], out)
    assert out.tolist() == c["expected"]


@pytest.mark.parametrize("kind,offset", [(Q4_K, 0), (Q4_K, 32), (Q4_K, 6), (Q6_K, 2), (Q6_K, 34), (Q8_0, 18)])
def test_mapped_and_owned_matvec_at_offsets(ctx, kind, offset):
    rows, cols = 40, 1024
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(30 + offset))
    x = synth.normal(synth.activation_seed(30 + offset), cols)
    want = capi.matvec(kind, rows, cols, w, x)
    blob = np.concatenate([np.full(offset, 0xAB, np.uint8), w, np.full(7, 0xCD, np.uint8)])
    mapping = ctx.map_read_only(blob)
    got = np.zeros(rows, np.float32)
    ctx.matvec_mapped(kind, rows, cols, mapping, offset, w.size, x, got)
    assert_close(got, want, "mapped")
    owned = ctx.new_owned_buffer(blob.size)
    owned.write(0, blob)
    got2 = np.zeros(rows, np.float32)
    ctx.matvec_owned(kind, rows, cols, owned, offset, w.size, x, got2)
    assert np.array_equal(bits(got), bits(got2))


def test_matvec_validation_mirrors_prepare_matvec(ctx):
    x = np.zeros(256, np.float32)
    enc = np.zeros(144, np.uint8)
    out = np.zeros(1, np.float32)
    cases = [
        (lambda: ctx.matvec(Q4_K, 1, 256, enc, x[:10], out), "InvalidInputLength"),
        (lambda: ctx.matvec(Q4_K, 1, 256, enc, x, np.zeros(2, np.float32)), "InvalidOutputLength"),
        (lambda: ctx.matvec(13, 1, 256, np.zeros(176, np.uint8), x, out), "UnsupportedTensorType"),
        (lambda: ctx.matvec(Q4_K, 1, 100, enc, x[:100], out), "InvalidElementCount"),
        (lambda: ctx.matvec(Q4_K, 1, 256, enc[:100], x, out), "InvalidByteLength"),
    ]
    for fn, variant in cases:
        with pytest.raises(HipError) as e:
            fn()
        assert e.value.variant == variant
    mapping = ctx.map_read_only(enc)
    with pytest.raises(HipError) as e:
        ctx.matvec_mapped(Q4_K, 1, 256, mapping, 8, 144, x, out)
    assert e.value.variant == "MappedRange"
    ctx.matvec(Q4_K, 0, 256, enc[:0], x, np.zeros(0, np.float32))  # rows == 0 is Ok


def test_seeded_golden_vectors(ctx, golden):
    _, seeded = golden
    for name in ("q4_k", "q6_k", "q8_0", "q6_k_768"):
        kind, rows, cols = (int(v) for v in seeded[f"{name}_shape"])
        enc = seeded[f"{name}_encoded"]
        buf = ctx.map_read_only(enc)
        deq = ctx.dequantize(kind, buf, 0, enc.size, rows * cols)
        assert int(bits(deq).astype(np.uint64).sum()) == int(seeded[f"{name}_dequant_checksum"][0]), name
        got = np.zeros(rows, np.float32)
        ctx.matvec_mapped(kind, rows, cols, buf, 0, enc.size, seeded[f"{name}_input"], got)
        assert_close(got, seeded[f"{name}_matvec"], name)


# ---- batch-1 decode GEMV at BASELINE shapes -------------------------------

@pytest.mark.parametrize("kind,rows,cols,cfg", [(Q4_K, 4096, 4096, 1), (Q6_K, 4096, 12288, 3),
                                                (Q4_K, 1536, 2048, 4), (Q6_K, 2048, 768, 4),
                                                (Q8_0, 4096, 4096, 6), (Q4_K, 12288, 4096, 3)])
def test_decode_gemv_matches_oracle(ctx, kind, rows, cols, cfg):
    print(f"gemv type={kind} {rows}x{cols}", flush=True)
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(cfg, 7))
    x = synth.normal(synth.activation_seed(cfg, 7), cols)
    want = capi.matvec(kind, rows, cols, w, x)
    wb, xb, yb = dev(ctx, w), dev(ctx, x), dev_out(ctx, rows * 4)
    ctx.matvec_device(kind, rows, cols, wb.device_ptr, 1, xb.device_ptr, yb.device_ptr)
    got = yb.read(0, rows * 4, np.float32)
    e, c = assert_close(got, want, f"{rows}x{cols}")
    exact, scale = exact_products(kind, rows, cols, w, x)
    ch = assert_channel_close(got, exact, scale, CHANNEL_TOL_GEMV, f"{rows}x{cols}")
    print(f"  rel_err={e:.2e} cosine={c:.9f} channel={ch:.2e} (oracle {channel_err(want, exact, scale):.2e})",
          flush=True)


@pytest.mark.parametrize("batch", [2, 3, 4, 8, 9, 16])
def test_batched_gemv_matches_oracle(ctx, batch):
    """Batches 1-4 take the int8 kernel at this size (records of every token
    in LDS), larger ones the fp16 kernel."""
    rows, cols = 1000, 2048
    for kind in (Q4_K, Q6_K):
        w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(40 + batch))
        x = synth.normal(synth.activation_seed(40 + batch), batch * cols).reshape(batch, cols)
        x[1 % batch] *= np.float32(1e-3)  # tokens of very different scale
        want = np.stack([capi.matvec(kind, rows, cols, w, x[b]) for b in range(batch)])
        wb, xb, yb = dev(ctx, w), dev(ctx, x), dev_out(ctx, batch * rows * 4)
        ctx.matvec_device(kind, rows, cols, wb.device_ptr, batch, xb.device_ptr, yb.device_ptr)
        got = yb.read(0, batch * rows * 4, np.float32).reshape(batch, rows)
        exact, scale = exact_products(kind, rows, cols, w, x)
        for b in range(batch):
            assert_close(got[b], want[b], f"type {kind} batch {batch} token {b}")
            assert_channel_close(got[b], exact[b], scale[b], CHANNEL_TOL_GEMV, f"type {kind} token {b}")


@pytest.mark.parametrize("kind,rows,cols,batch", [
    (Q6_K, 2048, 768, 4),    # 630-byte rows (every other row 2 bytes off a dword), odd block count
    (Q6_K, 300, 12288, 8),   # short and wide: K split over 8 waves, partial last tile
    (Q4_K, 100, 12288, 12),  # two token groups, partial tile
    (Q4_K, 4096, 12288, 3),  # fp16: above the size the int8 kernel takes 3-4 tokens for
    (Q4_K, 1000, 12288, 3),  # int8: three tokens' records of 48 blocks (117 KB of LDS)
    (Q6_K, 1000, 2560, 5),   # 10 blocks: partial last pair of a split
    (Q6_K, 300, 12288, 4),   # records too large for LDS: the fp16 kernel at 4 tokens
    (Q4_K, 70, 4096, 4),     # int8, 4 tokens, partial last tile
])
def test_batched_gemv_short_and_misaligned_shapes(ctx, kind, rows, cols, batch):
    """Batches above 2 on the int8 kernel (1-4 tokens whose records fit the
    LDS: misaligned 630-byte Q6_K rows, wide rows) and on the fp16 kernel's
    wide K split and partial block pairs."""
    print(f"batched gemv type={kind} {rows}x{cols} batch={batch}", flush=True)
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(90 + batch))
    x = synth.normal(synth.activation_seed(90 + batch), batch * cols).reshape(batch, cols)
    want = np.stack([capi.matvec(kind, rows, cols, w, x[b]) for b in range(batch)])
    wb, xb, yb = dev(ctx, w), dev(ctx, x), dev_out(ctx, batch * rows * 4)
    ctx.matvec_device(kind, rows, cols, wb.device_ptr, batch, xb.device_ptr, yb.device_ptr)
    got = yb.read(0, batch * rows * 4, np.float32).reshape(batch, rows)
    exact, scale = exact_products(kind, rows, cols, w, x)
    for b in range(batch):
        assert_close(got[b], want[b], f"type {kind} {rows}x{cols} batch {batch} token {b}")
        assert_channel_close(got[b], exact[b], scale[b], CHANNEL_TOL_GEMV, f"token {b}")


@pytest.mark.parametrize("kind,rows,cols,x_stride", [(Q4_K, 1000, 2048, 0), (Q6_K, 1000, 2048, 2048),
                                                     (Q4_K, 4096, 4096, 0), (Q8_0, 300, 512, 512)])
def test_matvec_batch_matches_one_matvec_per_matrix(ctx, kind, rows, cols, x_stride):
    """One grouped launch over 5 matrices (shared or per-matrix x, strided y)
    against the oracle per matrix; Q8_0 takes the per-matrix fallback."""
    count, y_stride = 5, rows + 24
    print(f"matvec batch type={kind} {rows}x{cols} x_stride={x_stride}", flush=True)
    ws = [synth.quantized_matrix(kind, rows, cols, synth.weight_seed(70 + i)) for i in range(count)]
    xs = synth.normal(synth.activation_seed(70), max(x_stride * (count - 1), 0) + cols)
    bufs = [dev(ctx, w) for w in ws]
    xb, yb = dev(ctx, xs), dev_out(ctx, count * y_stride * 4)
    yb.write(0, np.full(count * y_stride, -7.0, np.float32))
    ctx.matvec_batch_device(kind, rows, cols, [b.device_ptr for b in bufs], xb.device_ptr, x_stride,
                            yb.device_ptr, y_stride)
    got = yb.read(0, count * y_stride * 4, np.float32).reshape(count, y_stride)
    for i in range(count):
        x = xs[i * x_stride:i * x_stride + cols]
        assert_close(got[i, :rows], capi.matvec(kind, rows, cols, ws[i], x), f"matrix {i}")
        assert (got[i, rows:] == -7.0).all(), f"matrix {i} wrote past its rows"


def test_matvec_batch_validation(ctx):
    wb, xb, yb = dev_out(ctx, 144 * 8), dev_out(ctx, 1024), dev_out(ctx, 64)
    ctx.matvec_batch_device(Q4_K, 8, 256, [], xb.device_ptr, 0, yb.device_ptr, 8)  # no matrices: no-op
    with pytest.raises(HipError, match="InvalidArgument"):
        ctx.matvec_batch_device(Q4_K, 8, 256, [wb.device_ptr, 0], xb.device_ptr, 0, yb.device_ptr, 8)
    with pytest.raises(HipError, match="InvalidElementCount"):
        ctx.matvec_batch_device(Q4_K, 8, 100, [wb.device_ptr], xb.device_ptr, 0, yb.device_ptr, 8)


def _outlier_activations(seed, count, spikes=1e4):
    """N(0,1) values with, in every 256-value block, one element `spikes`
    times larger than its neighbours (random place and sign), and every
    seventh block scaled down by 1e-4 (small blocks beside large ones)."""
    x = synth.normal(synth.activation_seed(seed), count).astype(np.float64)
    rng = np.random.default_rng(seed)
    blocks = count // 256
    place = rng.integers(0, 256, blocks)
    sign = rng.choice([-1.0, 1.0], blocks)
    for b in range(blocks):
        if b % 7 == 3:
            x[256 * b:256 * b + 256] *= 1e-4
        else:
            x[256 * b + place[b]] = sign[b] * spikes * (1.0 + abs(x[256 * b + place[b]]))
    return x.astype(np.float32)


def _int8_record_bound(kind, rows, cols, w, x):
    """The int8 path's worst-case error per output row: each 256-value block
    of x is rounded to integers of 22 bits relative to the block's largest
    element, so |x~ - x| <= 2^-22 max_block|x|, and row r's error is at most
    sum over blocks of 2^-22 max_block|x| sum_block |W[r]| (fp32 rounding of
    the per-block sums adds a few ulp of the result on top)."""
    dense = capi.dequantize(kind, w, rows * cols).reshape(rows, cols).astype(np.float64)
    ax = np.abs(x.astype(np.float64))
    xb = ax.reshape(-1, 256).max(axis=1) * 2.0 ** -22
    wb = np.abs(dense).reshape(rows, -1, 256).sum(axis=2)
    # plus the fp32 summation noise of the reference's sequential fold
    # (random-walk size, 8 sqrt(cols) ulp of sum |W x|)
    noise = 8.0 * np.sqrt(cols) * np.finfo(np.float32).eps * (np.abs(dense) @ ax)
    return wb @ xb + noise


def _fp16_pair_bound(kind, rows, cols, w, x):
    """The fp16 path's worst-case error per output row (batches 3-16): the
    token is scaled by one power of two so max|x| 2^-e lies in [2^14, 2^15)
    and split into fp16 hi + lo, so |x~ - x| <= 2^-22 |x| (two roundings of
    half an fp16 ulp) + 2^-39 max|x| (lo below fp16's normal range).  Q4_K's
    dmin m sum(x) term takes 32-column sums in fp32 (at most 31 roundings,
    2^-19 of sum|x|) before the same split, and dmin m <= 63 dmin bounds its
    factor.  The fp32 noise term is the one of the int8 bound."""
    dense = capi.dequantize(kind, w, rows * cols).reshape(rows, cols).astype(np.float64)
    ax = np.abs(x.astype(np.float64))
    per_x = 2.0 ** -22 * ax + 2.0 ** -39 * ax.max()
    bound = np.abs(dense) @ per_x
    if kind == Q4_K:
        blocks = w.reshape(rows, cols // 256, 144)
        dmin = blocks[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
        sub = ax.reshape(-1, 32).sum(axis=1).reshape(cols // 256, 8).sum(axis=1)
        bound += (63.0 * dmin * (2.0 ** -19 + 2.0 ** -22)) @ sub
    noise = 8.0 * np.sqrt(cols) * np.finfo(np.float32).eps * (np.abs(dense) @ ax)
    return bound + noise


@pytest.mark.parametrize("kind,rows,cols,batch", [(Q4_K, 4096, 4096, 1), (Q6_K, 4096, 4096, 2),
                                                 (Q8_0, 4096, 4096, 1), (Q4_K, 1000, 2048, 4),
                                                 (Q6_K, 1000, 2048, 8), (Q4_K, 1000, 2048, 8),
                                                 (Q4_K, 4096, 12288, 6)])
def test_in_block_outliers_stay_within_the_bound(ctx, kind, rows, cols, batch):
    """One element 10^4 times its neighbours inside each 256-value block, and
    blocks 10^4 smaller than the rest: batches of 1-4 tokens take the int8
    records (22 bits per block), batches 6 and 8 the fp16 path (22 bits per
    token); each is checked against the bound derived for its path, and the
    tolerance."""
    print(f"outliers type={kind} {rows}x{cols} batch={batch}", flush=True)
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(130, kind))
    x = np.stack([_outlier_activations(131 + b, cols) for b in range(batch)])
    want = np.stack([capi.matvec(kind, rows, cols, w, x[b]) for b in range(batch)])
    wb, xb, yb = dev(ctx, w), dev(ctx, x), dev_out(ctx, batch * rows * 4)
    ctx.matvec_device(kind, rows, cols, wb.device_ptr, batch, xb.device_ptr, yb.device_ptr)
    got = yb.read(0, batch * rows * 4, np.float32).reshape(batch, rows)
    for b in range(batch):
        e, _ = assert_close(got[b], want[b], f"outliers type {kind} token {b}")
        if batch <= 4:
            bound = _int8_record_bound(kind, rows, cols, w, x[b])
        else:
            bound = _fp16_pair_bound(kind, rows, cols, w, x[b])
        err = np.abs(got[b].astype(np.float64) - want[b])
        assert (err <= bound).all(), f"token {b}: worst excess {np.max(err - bound):.3g}"
        print(f"  token {b}: rel_err={e:.2e} worst err/bound={float((err / bound).max()):.3f}", flush=True)


@pytest.mark.parametrize("kind", [Q6_K, Q4_K])
def test_argmax_with_in_block_outliers(ctx, kind):
    """The fused argmax on outlier activations: the index equals the CPU's
    whenever the CPU's top-2 gap exceeds twice the int8 path's error bound
    (and always equals the argmax of the GPU's own logits)."""
    rows, cols = 30000, 4096
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(132, kind))
    x = _outlier_activations(133, cols)
    want = capi.matvec(kind, rows, cols, w, x)
    wb, xb, yb, ib = dev(ctx, w), dev(ctx, x), dev_out(ctx, rows * 4), dev_out(ctx, 4)
    ctx.matvec_argmax_device(kind, rows, cols, wb.device_ptr, xb.device_ptr, yb.device_ptr, ib.device_ptr)
    idx = ctx.argmax_result()
    got = yb.read(0, rows * 4, np.float32)
    assert_close(got, want, "outlier logits")
    assert idx == capi.argmax(got)
    bound = _int8_record_bound(kind, rows, cols, w, x).max()
    gap = top2_gap(want)
    print(f"  argmax gpu={idx} cpu={capi.argmax(want)} gap={gap:.4g} bound={bound:.3g}", flush=True)
    if gap > 2 * bound:
        assert idx == capi.argmax(want)


@pytest.mark.parametrize("kind", [Q4_K, Q6_K, Q8_0])
def test_prefill_gemm_with_in_block_outliers(ctx, kind):
    """The GEMM's A preparation scales each K quarter of a row by one power of
    two: outliers 10^4 times their neighbours and blocks 10^4 smaller than the
    rest (bf16 values down to 2^-17 of the quarter's maximum convert to fp16
    exactly)."""
    m, n, k = 160, 192, 4096
    a = synth.to_bf16_bits(np.concatenate([_outlier_activations(140 + r, k) for r in range(m)]))
    w = synth.quantized_matrix(kind, n, k, synth.weight_seed(141, kind))
    want = capi.gemm_tokenwise(kind, m, n, k, a, w)
    ab, wb, cb = dev(ctx, a), dev(ctx, w), dev_out(ctx, m * n * 4)
    ws = dev_out(ctx, ctx.gemm_workspace_bytes(m, k))
    ctx.gemm_device(kind, m, n, k, ab.device_ptr, wb.device_ptr, cb.device_ptr, ws.device_ptr, len(ws))
    got = cb.read(0, m * n * 4, np.float32).reshape(m, n)
    worst = 0.0
    for r in range(m):
        e, _ = assert_close(got[r], want[r], f"outlier GEMM type {kind} token {r}")
        worst = max(worst, e)
    print(f"  type {kind}: worst rel_err={worst:.2e}", flush=True)


_SMALL_D = (1e-6, 1e-5, 3e-5)


def _small_scale_matrix(kind, rows, cols, seed):
    """Seeded blocks whose super-block scale d is replaced by 1e-6, 1e-5 or
    3e-5 (fp16 subnormals: 17, 168 and 503 times 2^-24) on rows 4j, 4j + 1
    and 4j + 2, and by 1e-6 on the even blocks of rows 4j + 3, beside rows
    of the seeded scales; Q4_K's dmin becomes half the new d.  Such rows are
    30 to 2000 times smaller than their neighbours, so the per-channel
    measure sees them where the vector-wide one would not."""
    w = synth.quantized_matrix(kind, rows, cols, seed).copy()
    elems, nbytes = synth.BLOCK[kind]
    blk = w.reshape(rows, cols // elems, nbytes)
    d_at = {Q4_K: 0, Q6_K: 208, Q8_0: 0}[kind]

    def put(part, dv):
        part[..., d_at:d_at + 2] = np.float16([dv]).view(np.uint8)
        if kind == Q4_K:
            part[..., 2:4] = np.float16([dv / 2]).view(np.uint8)

    for j, dv in enumerate(_SMALL_D):
        put(blk[j::4], dv)
    put(blk[3::4, 0::2], _SMALL_D[0])
    return w


@pytest.mark.parametrize("kind", [Q4_K, Q6_K, Q8_0])
@pytest.mark.parametrize("batch", [1, 2, 4, 8])
def test_small_scale_blocks_gemv(ctx, kind, batch):
    """Super-block scales in fp16's subnormal range beside ordinary rows: the
    int8 records (batch 1-4) and the fp16 pairs (batch 8) keep every output
    channel within the per-channel bar, not only the vector-wide one."""
    rows, cols = 4096, 4096
    w = _small_scale_matrix(kind, rows, cols, synth.weight_seed(150, kind))
    x = synth.normal(synth.activation_seed(150, batch), batch * cols).reshape(batch, cols)
    want = np.stack([capi.matvec(kind, rows, cols, w, x[b]) for b in range(batch)])
    wb, xb, yb = dev(ctx, w), dev(ctx, x), dev_out(ctx, batch * rows * 4)
    ctx.matvec_device(kind, rows, cols, wb.device_ptr, batch, xb.device_ptr, yb.device_ptr)
    got = yb.read(0, batch * rows * 4, np.float32).reshape(batch, rows)
    exact, scale = exact_products(kind, rows, cols, w, x)
    worst = 0.0
    for b in range(batch):
        assert_close(got[b], want[b], f"small scales type {kind} token {b}")
        worst = max(worst, assert_channel_close(got[b], exact[b], scale[b], CHANNEL_TOL_GEMV,
                                                f"small scales type {kind} token {b}"))
        small = np.arange(rows) % 4 == 0  # the d = 1e-6 rows alone
        assert channel_err(got[b][small], exact[b][small], scale[b][small]) <= CHANNEL_TOL_GEMV
    print(f"  type {kind} batch {batch}: channel={worst:.2e}", flush=True)


@pytest.mark.parametrize("kind", [Q4_K, Q6_K, Q8_0])
def test_small_scale_blocks_gemm(ctx, kind):
    """The GEMM's fp16 weight factors at subnormal super-block scales: d is
    itself an fp16 value, so d sc (Q4_K, Q6_K), dmin m and every weight
    below 2^-14 lie on fp16's 2^-24 grid and convert exactly; above it one
    rounding of 2^-11 applies as for any other block.  Every token's
    channels stay within the GEMM's per-channel bar."""
    m, n, k = 160, 256, 4096
    a = synth.to_bf16_bits(synth.normal(synth.activation_seed(151, kind), m * k))
    w = _small_scale_matrix(kind, n, k, synth.weight_seed(151, kind))
    want = capi.gemm_tokenwise(kind, m, n, k, a, w)
    ab, wb, cb = dev(ctx, a), dev(ctx, w), dev_out(ctx, m * n * 4)
    ws = dev_out(ctx, ctx.gemm_workspace_bytes(m, k))
    ctx.gemm_device(kind, m, n, k, ab.device_ptr, wb.device_ptr, cb.device_ptr, ws.device_ptr, len(ws))
    got = cb.read(0, m * n * 4, np.float32).reshape(m, n)
    for r in range(m):
        assert_close(got[r], want[r], f"small-scale GEMM type {kind} token {r}")
    exact, scale = exact_products(kind, n, k, w, synth.bf16_bits_to_f32(a).reshape(m, k))
    ch = assert_channel_close(got, exact, scale, CHANNEL_TOL_GEMM, f"small-scale GEMM type {kind}")
    small = np.arange(n) % 4 == 0
    ch_small = channel_err(got[:, small], exact[:, small], scale[:, small])
    assert ch_small <= CHANNEL_TOL_GEMM
    print(f"  type {kind}: channel={ch:.2e} (d = 1e-6 rows {ch_small:.2e})", flush=True)


def test_q6_k_large_scales_take_the_exact_split_path(ctx):
    rows, cols = 64, 1024
    w = synth.quantized_matrix(Q6_K, rows, cols, synth.weight_seed(55)).reshape(-1, 210).copy()
    rng = np.random.default_rng(1)
    w[::3, 192:208] = rng.integers(-128, 128, size=(w[::3].shape[0], 16)).astype(np.int8).view(np.uint8)
    w = w.reshape(-1)
    x = synth.normal(56, cols)
    want = capi.matvec(Q6_K, rows, cols, w, x)
    wb, xb, yb = dev(ctx, w), dev(ctx, x), dev_out(ctx, rows * 4)
    ctx.matvec_device(Q6_K, rows, cols, wb.device_ptr, 1, xb.device_ptr, yb.device_ptr)
    assert_close(yb.read(0, rows * 4, np.float32), want, "large Q6_K scales")


def test_output_head_q6_k_with_argmax(ctx):
    """Config 2: Q6_K 151936 x 4096 plus greedy argmax (bit-exact index)."""
    rows, cols = 151936, 4096
    print("C2 generate", flush=True)
    w = synth.quantized_matrix(Q6_K, rows, cols, synth.weight_seed(2))
    x = synth.normal(synth.activation_seed(2), cols)
    want = capi.matvec(Q6_K, rows, cols, w, x)
    want_idx = capi.argmax(want)
    wb, xb, yb, ib = dev(ctx, w), dev(ctx, x), dev_out(ctx, rows * 4), dev_out(ctx, 4)
    print("C2 run", flush=True)
    ctx.matvec_argmax_device(Q6_K, rows, cols, wb.device_ptr, xb.device_ptr, yb.device_ptr, ib.device_ptr)
    idx = ctx.argmax_result()
    got = yb.read(0, rows * 4, np.float32)
    assert_close(got, want, "C2 logits")
    exact, scale = exact_products(Q6_K, rows, cols, w, x)
    ch = assert_channel_close(got, exact, scale, CHANNEL_TOL_GEMV, "C2 logits")
    print(f"  channel={ch:.2e} (oracle {channel_err(want, exact, scale):.2e})", flush=True)
    assert idx == capi.argmax(got)  # the fused argmax is exact on the GPU's logits
    gap = top2_gap(want)
    print(f"  argmax gpu={idx} cpu={want_idx} top2 gap={gap:.4g}", flush=True)
    assert idx == want_idx


@pytest.mark.parametrize("kind,rows,cols,batch", [(Q4_K, 70000, 4096, 1), (Q6_K, 66001, 2048, 2),
                                                 (Q6_K, 65600, 768, 1), (Q4_K, 66000, 12288, 1),
                                                 (Q4_K, 40007, 4096, 2), (Q8_0, 36001, 2048, 2),
                                                 (Q8_0, 33000, 12288, 1), (Q4_K, 140001, 2048, 2),
                                                 (Q8_0, 131089, 4096, 1)])
def test_tall_matvec_persistent_plans(ctx, kind, rows, cols, batch):
    """Tall matrices take the persistent plans: waves that each stream their
    own tiles, and for 8192 tiles or more of Q4_K and Q8_0 workgroups whose
    8 waves share each tile.  Row counts that end mid-tile, three-block and
    wide rows, two tokens."""
    print(f"tall type={kind} {rows}x{cols} batch={batch}", flush=True)
    w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(60, rows))
    x = synth.normal(synth.activation_seed(60, rows), batch * cols).reshape(batch, cols)
    wb, xb, yb = dev(ctx, w), dev(ctx, x), dev_out(ctx, batch * rows * 4)
    ctx.matvec_device(kind, rows, cols, wb.device_ptr, batch, xb.device_ptr, yb.device_ptr)
    got = yb.read(0, batch * rows * 4, np.float32).reshape(batch, rows)
    for b in range(batch):
        assert_close(got[b], capi.matvec(kind, rows, cols, w, x[b]), f"token {b}")
    if batch == 1:
        ib = dev_out(ctx, 4)
        ctx.matvec_argmax_device(kind, rows, cols, wb.device_ptr, xb.device_ptr, yb.device_ptr, ib.device_ptr)
        assert ctx.argmax_result() == capi.argmax(yb.read(0, rows * 4, np.float32))


def test_softcap_matches_the_reference_fixture(ctx):
    """MetalContext::softcap (src/metal.rs:600-622) on the reference's own
    fixture (src/metal.rs:2166-2168, 2231-2235: 513 values, cap 30, absolute
    tolerance 2e-6), a wide range of magnitudes, the device form in place,
    and the reference's check order."""
    fixture = np.array([((i % 31) - 15) * 0.071 for i in range(513)], dtype=np.float32)
    out = np.zeros(513, dtype=np.float32)
    ctx.softcap(fixture, 30.0, out)
    assert np.abs(out - capi.softcap(fixture, 30.0)).max() <= 2.0e-6
    wide = np.concatenate([synth.normal(synth.activation_seed(150), 4000) * np.float32(20.0),
                           np.float32([0.0, -0.0, 1e-30, 1e4, -1e4, 3.4e38, -3.4e38])])
    for cap in (30.0, 1.5):
        out = np.zeros(wide.size, dtype=np.float32)
        ctx.softcap(wide, cap, out)
        want = capi.softcap(wide, cap).astype(np.float64)
        ulp = np.spacing(np.maximum(np.abs(want), 1e-38).astype(np.float32)).astype(np.float64)
        assert (np.abs(out - want) <= 4 * ulp).all(), cap
    buf = dev(ctx, wide)
    ctx.softcap_device(wide.size, buf.device_ptr, 30.0, buf.device_ptr)
    np.testing.assert_allclose(buf.read(0, wide.size * 4, np.float32), capi.softcap(wide, 30.0), rtol=0, atol=1e-4)
    for args, variant in (((np.zeros(0, np.float32), -1.0, np.zeros(0, np.float32)), "EmptyInput"),
                          ((fixture, -1.0, np.zeros(3, np.float32)), "InvalidVectorLength"),
                          ((fixture, 0.0, np.zeros(513, np.float32)), "InvalidPositiveParameter"),
                          ((fixture, float("nan"), np.zeros(513, np.float32)), "InvalidPositiveParameter")):
        with pytest.raises(HipError) as e:
            ctx.softcap(*args)
        assert e.value.variant == variant


@pytest.mark.parametrize("rows,cols,batch", [(1000, 2048, 1), (4096, 4096, 2), (300, 12288, 1), (40000, 4096, 1),
                                             (513, 4128, 1), (700, 2048, 5), (513, 4128, 3), (700, 2048, 3),
                                             (4096, 4096, 4), (300, 12288, 6)])
def test_q8_0_gemv_matches_oracle(ctx, rows, cols, batch):
    """Q8_0 on the int8 kernel (whole 8-block super-blocks; up to 4 tokens a
    launch, fewer when their records do not fit the LDS, larger batches as
    several launches); 4128 columns (129 blocks) take the exact per-element
    kernel."""
    print(f"Q8_0 gemv {rows}x{cols} batch={batch}", flush=True)
    w = synth.quantized_matrix(Q8_0, rows, cols, synth.weight_seed(80 + batch))
    x = synth.normal(synth.activation_seed(80 + batch), batch * cols).reshape(batch, cols)
    want = np.stack([capi.matvec(Q8_0, rows, cols, w, x[b]) for b in range(batch)])
    wb, xb, yb = dev(ctx, w), dev(ctx, x), dev_out(ctx, batch * rows * 4)
    ctx.matvec_device(Q8_0, rows, cols, wb.device_ptr, batch, xb.device_ptr, yb.device_ptr)
    got = yb.read(0, batch * rows * 4, np.float32).reshape(batch, rows)
    for b in range(batch):
        assert_close(got[b], want[b], f"Q8_0 {rows}x{cols} token {b}")


@pytest.mark.parametrize("kind,rows", [(Q6_K, 48000), (Q4_K, 48000), (Q4_K, 140000), (Q8_0, 140000)])
def test_fused_argmax_ties_resolve_to_the_lowest_row(ctx, kind, rows):
    """Rows repeat with period 97, so the maximum appears in hundreds of rows
    spread over many workgroups: the device-wide key maximum must return the
    first of them (src/cpu.rs:275-293 keeps the first maximum).  140000 rows
    take the workgroups that share each tile (Q4_K, Q8_0)."""
    cols, period = 4096, 97
    base = synth.quantized_matrix(kind, period, cols, synth.weight_seed(97, kind))
    rb = base.size // period
    w = np.concatenate([base.reshape(period, rb)] * (rows // period + 1))[:rows].reshape(-1)
    x = synth.normal(synth.activation_seed(97), cols)
    wb, xb, yb, ib = dev(ctx, w), dev(ctx, x), dev_out(ctx, rows * 4), dev_out(ctx, 4)
    ctx.matvec_argmax_device(kind, rows, cols, wb.device_ptr, xb.device_ptr, yb.device_ptr, ib.device_ptr)
    got = yb.read(0, rows * 4, np.float32)
    idx = ctx.argmax_result()
    want_row = capi.argmax(capi.matvec(kind, period, cols, base, x))
    assert idx == want_row == capi.argmax(got)
    assert np.count_nonzero(got == got[idx]) >= rows // period


@pytest.mark.parametrize("kind", [Q4_K, Q6_K, Q8_0])
def test_prefill_gemm_short_prefills_take_the_tokenwise_path(ctx, kind):
    """Up to 16 tokens run the decode GEMV (one pass over W per 16 tokens)."""
    m, n, k = 16, 96, 512
    a = synth.to_bf16_bits(synth.normal(synth.activation_seed(8, kind), m * k))
    w = synth.quantized_matrix(kind, n, k, synth.weight_seed(8, kind))
    want = capi.gemm_tokenwise(kind, m, n, k, a, w)
    ab, wb, cb = dev(ctx, a), dev(ctx, w), dev_out(ctx, m * n * 4)
    ws = dev_out(ctx, ctx.gemm_workspace_bytes(m, k))
    ctx.gemm_device(kind, m, n, k, ab.device_ptr, wb.device_ptr, cb.device_ptr, ws.device_ptr, len(ws))
    got = cb.read(0, m * n * 4, np.float32).reshape(m, n)
    for r in range(m):
        assert_close(got[r], want[r], f"type {kind} token {r}")


def test_q8_0_argmax_is_exact(ctx):
    rows, cols = 50000, 4096
    w = synth.quantized_matrix(Q8_0, rows, cols, synth.weight_seed(88))
    x = synth.normal(synth.activation_seed(88), cols)
    want = capi.matvec(Q8_0, rows, cols, w, x)
    wb, xb, yb, ib = dev(ctx, w), dev(ctx, x), dev_out(ctx, rows * 4), dev_out(ctx, 4)
    ctx.matvec_argmax_device(Q8_0, rows, cols, wb.device_ptr, xb.device_ptr, yb.device_ptr, ib.device_ptr)
    idx = ctx.argmax_result()
    got = yb.read(0, rows * 4, np.float32)
    assert_close(got, want, "Q8_0 logits")
    assert idx == capi.argmax(got)
    print(f"  argmax gpu={idx} cpu={capi.argmax(want)} top2 gap={top2_gap(want):.4g}", flush=True)
    assert idx == capi.argmax(want)


def test_argmax_fused_rejects_non_finite(ctx):
    rows, cols = 300, 256
    w = synth.quantized_matrix(Q6_K, rows, cols, 3)
    x = synth.normal(4, cols)
    x[7] = np.inf
    wb, xb, yb, ib = dev(ctx, w), dev(ctx, x), dev_out(ctx, rows * 4), dev_out(ctx, 4)
    ctx.matvec_argmax_device(Q6_K, rows, cols, wb.device_ptr, xb.device_ptr, yb.device_ptr, ib.device_ptr)
    with pytest.raises(HipError) as e:
        ctx.argmax_result()
    assert e.value.variant == "NonFinite"
    # The fused finish leaves its device-wide maximum and ticket reset: the
    # next calls on the context see only their own rows.
    for seed in (5, 6):
        x = synth.normal(seed, cols)
        xb = dev(ctx, x)
        ctx.matvec_argmax_device(Q6_K, rows, cols, wb.device_ptr, xb.device_ptr, yb.device_ptr, ib.device_ptr)
        idx = ctx.argmax_result()
        assert idx == capi.argmax(yb.read(0, rows * 4, np.float32))
        assert idx == capi.argmax(capi.matvec(Q6_K, rows, cols, w, x))


# ---- reductions and activations ------------------------------------------

def test_argmax_top_k_rms_norm_silu(ctx, golden):
    kat, seeded = golden
    assert ctx.argmax(kat["argmax_ties"]["input"]) == kat["argmax_ties"]["expected"]
    assert ctx.argmax([-0.0, 0.0]) == 1
    c = kat["top_k"]
    sel = ctx.top_k_softmax(c["logits"], c["k"])
    assert [s[0] for s in sel] == [e[0] for e in c["expected"]]
    assert np.allclose([s[1] for s in sel], [e[1] for e in c["expected"]], rtol=1e-6)
    sel = ctx.top_k_softmax(seeded["top_k_logits"], 8)
    assert [s[0] for s in sel] == seeded["top_k_ids"].tolist()
    assert np.allclose([s[1] for s in sel], seeded["top_k_probs"], rtol=1e-5)
    for bad, variant in (([], "EmptyInput"), ([1.0, np.nan], "NonFinite")):
        with pytest.raises(HipError) as e:
            ctx.argmax(bad)
        assert e.value.variant == variant
    with pytest.raises(HipError) as e:
        ctx.top_k_softmax([1.0], 0)
    assert e.value.variant == "InvalidTopK"
    big = synth.normal(90, 200003)
    assert ctx.argmax(big) == capi.argmax(big)
    c = kat["rms_norm"]
    out = np.zeros(2, np.float32)
    ctx.rms_norm(c["input"], None, c["epsilon"], out)
    assert np.array_equal(bits(out), bits(c["expected_unweighted"]))
    ctx.rms_norm(c["input"], c["weight"], c["epsilon"], out)
    assert np.array_equal(bits(out), bits(c["expected_weighted"]))
    with pytest.raises(HipError) as e:
        ctx.rms_norm(c["input"], c["bad_weight"], c["epsilon"], out)
    assert e.value.variant == "InvalidVectorLength"
    v = synth.normal(91, 4096)
    out = np.zeros(4096, np.float32)
    ctx.rms_norm(v, None, 1e-6, out)
    assert_close(out, capi.rms_norm(v, None, 1e-6), "rms_norm")
    g, u = synth.normal(92, 5000) * 4, synth.normal(93, 5000)
    out = np.zeros(5000, np.float32)
    ctx.silu_mul(g, u, out)
    want = np.array([capi.silu(float(a)) for a in g], np.float32) * u
    assert_close(out, want, "silu_mul")


# ---- config 3: dense FFN at decode ----------------------------------------

@pytest.mark.parametrize("batch", [1, 2, 3, 4, 8])
def test_dense_ffn_matches_oracle(ctx, batch):
    """Config 3.  Batch 1-2 runs the int8 gate/up kernel with RMSNorm folded
    into its activation scale, batches 3-8 the fp16 one; the down projection
    (12288 columns) is int8 for 1-2 tokens and fp16 above."""
    hidden, ffn = 4096, 12288
    print(f"C3 batch={batch}", flush=True)
    g = synth.quantized_matrix(Q4_K, ffn, hidden, synth.weight_seed(3, 0))
    u = synth.quantized_matrix(Q4_K, ffn, hidden, synth.weight_seed(3, 1))
    d = synth.quantized_matrix(Q6_K, hidden, ffn, synth.weight_seed(3, 2))
    h = synth.normal(synth.activation_seed(3, batch), batch * hidden).reshape(batch, hidden)
    want = capi.dense_ffn(batch, hidden, ffn, Q4_K, g, Q4_K, u, Q6_K, d, h)
    gb, ub, db, hb = dev(ctx, g), dev(ctx, u), dev(ctx, d), dev(ctx, h)
    yb = dev_out(ctx, batch * hidden * 4)
    ws = dev_out(ctx, ctx.ffn_workspace_bytes(batch, hidden, ffn))
    ctx.ffn_device(batch, hidden, ffn, Q4_K, gb.device_ptr, Q4_K, ub.device_ptr, Q6_K, db.device_ptr,
                   1e-6, hb.device_ptr, yb.device_ptr, ws.device_ptr, len(ws))
    got = yb.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
    for b in range(batch):
        e, c = assert_close(got[b], want[b], f"C3 token {b}")
    print(f"  rel_err={e:.2e} cosine={c:.9f}", flush=True)


@pytest.mark.parametrize("gu_type,dn_type,batch", [(Q4_K, Q6_K, 2), (Q8_0, Q8_0, 2), (Q8_0, Q6_K, 1),
                                                    (Q4_K, Q4_K, 5)])
def test_ffn_wide_hidden_stays_inside_its_workspace(ctx, gu_type, dn_type, batch):
    """hidden = 8 * ffn: the workspace is allocated at exactly the advertised
    size with a guard region after it, which must come back unchanged; the
    fused (Q4_K pairs) and unfused (Q8_0 pairs) paths both match the oracle,
    and a workspace one byte short is rejected."""
    hidden, ffn = 2048, 256
    g = synth.quantized_matrix(gu_type, ffn, hidden, synth.weight_seed(33, 0))
    u = synth.quantized_matrix(gu_type, ffn, hidden, synth.weight_seed(33, 1))
    d = synth.quantized_matrix(dn_type, hidden, ffn, synth.weight_seed(33, 2))
    h = synth.normal(synth.activation_seed(33, batch), batch * hidden).reshape(batch, hidden)
    want = capi.dense_ffn(batch, hidden, ffn, gu_type, g, gu_type, u, dn_type, d, h)
    gb, ub, db, hb = dev(ctx, g), dev(ctx, u), dev(ctx, d), dev(ctx, h)
    yb = dev_out(ctx, batch * hidden * 4)
    need = ctx.ffn_workspace_bytes(batch, hidden, ffn)
    assert need >= batch * (hidden + 3 * ffn) * 4
    guard = 4096
    ws = dev_out(ctx, need + guard)
    ws.write(need, np.full(guard, 0xA5, np.uint8))
    ctx.ffn_device(batch, hidden, ffn, gu_type, gb.device_ptr, gu_type, ub.device_ptr, dn_type, db.device_ptr,
                   1e-6, hb.device_ptr, yb.device_ptr, ws.device_ptr, need)
    got = yb.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
    for b in range(batch):
        assert_close(got[b], want[b], f"token {b}")
    assert (ws.read(need, guard) == 0xA5).all(), "FFN wrote past its workspace"
    with pytest.raises(HipError) as e:
        ctx.ffn_device(batch, hidden, ffn, gu_type, gb.device_ptr, gu_type, ub.device_ptr, dn_type,
                       db.device_ptr, 1e-6, hb.device_ptr, yb.device_ptr, ws.device_ptr, need - 1)
    assert e.value.variant == "InvalidArgument"


# ---- config 4: routed experts ------------------------------------------------

def _moe_setup(hidden=2048, width=768, experts=128):
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(4, 9), experts * hidden) * np.float32(0.02))
    gu_row, dn_row = synth.row_bytes(Q4_K, hidden), synth.row_bytes(Q6_K, width)
    gu_bytes, dn_bytes = 2 * width * gu_row, hidden * dn_row
    gu = synth.quantized_matrix(Q4_K, experts * 2 * width, hidden, synth.weight_seed(4, 0))
    dn = synth.quantized_matrix(Q6_K, experts * hidden, width, synth.weight_seed(4, 1))
    return router, gu, dn, gu_bytes, dn_bytes


@pytest.mark.parametrize("batch,hidden,experts,k", [(1, 2048, 128, 8), (5, 2048, 128, 8), (2, 1000, 60, 4),
                                                    (3, 2824, 128, 8), (2, 4096, 256, 8), (2, 1016, 200, 6),
                                                    (1, 2050, 128, 8), (1, 512, 300, 8), (2, 1024, 12, 4),
                                                    (33, 2048, 128, 8), (4100, 256, 16, 2), (2, 24576, 128, 8),
                                                    (3, 4104, 64, 4), (2, 2048, 200, 6), (1, 2048, 16, 2),
                                                    (2, 2048, 256, 8), (4100, 2048, 48, 4)])
def test_router_top_k_is_bit_exact(ctx, batch, hidden, experts, k):
    """The bf16 router fold (src/cpu.rs:384-397 order) and top-k: logits bit
    for bit, ids exact.  Covers the expert-parallel fold at hidden 2048 (32
    rows per workgroup staged in LDS, partial last workgroups, 16 to 256
    experts), the expert-parallel fold at other widths (8 experts per
    workgroup, 512-column chunks, partial last chunks and workgroups, long
    rows; above 4096 tokens the selection runs as a second launch), the
    LDS-staged one-workgroup kernel (fewer than 16 experts), and the
    unstaged kernel (hidden % 8 != 0, more than 256 experts)."""
    print(f"router batch={batch} hidden={hidden} experts={experts} k={k}", flush=True)
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(6, hidden), experts * hidden) * np.float32(0.02))
    x = synth.normal(synth.activation_seed(6, experts), batch * hidden).reshape(batch, hidden)
    rb, xb = dev(ctx, router), dev(ctx, x)
    lb, ib, pb = dev_out(ctx, batch * experts * 4), dev_out(ctx, batch * k * 4), dev_out(ctx, batch * k * 4)
    ctx.router_top_k_device(batch, hidden, experts, k, rb.device_ptr, xb.device_ptr, lb.device_ptr,
                            ib.device_ptr, pb.device_ptr)
    logits = lb.read(0, batch * experts * 4, np.float32).reshape(batch, experts)
    ids = ib.read(0, batch * k * 4, np.uint32).reshape(batch, k)
    probs = pb.read(0, batch * k * 4, np.float32).reshape(batch, k)
    for t in range(batch):
        want = capi.matvec_bf16(experts, hidden, router, x[t])
        assert np.array_equal(bits(logits[t]), bits(want)), f"token {t} logits"
        top = capi.top_k_softmax(want, k)
        assert ids[t].tolist() == [e for e, _ in top]
        assert np.allclose(probs[t], [p for _, p in top], rtol=1e-6)


def test_router_rejects_non_finite_logits(ctx):
    """top_k_softmax rejects non-finite logits (src/cpu.rs:240-245): an Inf in
    a token makes dmhip_router_result report NonFinite, the next clean call
    reports nothing, and a result covers every call since the previous one."""
    batch, hidden, experts, k = 3, 2048, 128, 8
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(6, 1), experts * hidden) * np.float32(0.02))
    x = synth.normal(synth.activation_seed(6, 1), batch * hidden).reshape(batch, hidden)
    rb = dev(ctx, router)
    lb, ib, pb = dev_out(ctx, batch * experts * 4), dev_out(ctx, batch * k * 4), dev_out(ctx, batch * k * 4)
    bad = x.copy()
    bad[1, 77] = np.inf
    xb = dev(ctx, bad)
    ctx.router_top_k_device(batch, hidden, experts, k, rb.device_ptr, xb.device_ptr, lb.device_ptr, ib.device_ptr,
                            pb.device_ptr)
    with pytest.raises(HipError) as e:
        ctx.router_result()
    assert e.value.variant == "NonFinite"
    xb = dev(ctx, x)
    ctx.router_top_k_device(batch, hidden, experts, k, rb.device_ptr, xb.device_ptr, lb.device_ptr, ib.device_ptr,
                            pb.device_ptr)
    ctx.router_result()
    ids = ib.read(0, batch * k * 4, np.uint32).reshape(batch, k)
    for t in range(batch):
        want = capi.top_k_softmax(capi.matvec_bf16(experts, hidden, router, x[t]), k)
        assert ids[t].tolist() == [i for i, _ in want]
    # one result covers every call since the previous result: the bad call
    # first, then a clean one, is still reported
    xbad = dev(ctx, bad)
    for buf in (xbad, xb):
        ctx.router_top_k_device(batch, hidden, experts, k, rb.device_ptr, buf.device_ptr, lb.device_ptr,
                                ib.device_ptr, pb.device_ptr)
    with pytest.raises(HipError) as e:
        ctx.router_result()
    assert e.value.variant == "NonFinite"


@pytest.mark.parametrize("experts,hidden", [(128, 2048), (12, 1024), (300, 512)])
def test_moe_layer_rejects_non_finite_router_input(ctx, experts, hidden):
    """A non-finite token makes the layer return NonFinite before any expert
    is acquired (no cache counters move), for the expert-parallel router,
    the one-workgroup router (< 16 experts) and the fallback (> 256); a clean
    call afterwards succeeds."""
    width, k, batch = 256, 4, 2
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(44, experts), experts * hidden) * np.float32(0.02))
    gu_bytes, dn_bytes = 2 * width * synth.row_bytes(Q4_K, hidden), hidden * synth.row_bytes(Q6_K, width)
    gu = synth.quantized_matrix(Q4_K, experts * 2 * width, hidden, synth.weight_seed(44, 1))
    dn = synth.quantized_matrix(Q6_K, experts * hidden, width, synth.weight_seed(44, 2))
    src = np.concatenate([gu, dn])
    cache = ExpertCache(ctx, src, [ExpertLayerLayout(experts, 0, gu_bytes, gu.size, dn_bytes)], 4)
    x = synth.normal(synth.activation_seed(44, experts), batch * hidden).reshape(batch, hidden)
    bad = x.copy()
    bad[batch - 1, 3] = np.nan
    rb, yb = dev(ctx, router), dev_out(ctx, batch * hidden * 4)
    with pytest.raises(HipError) as e:
        ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                      dev(ctx, bad).device_ptr, yb.device_ptr)
    assert e.value.variant == "NonFinite"
    assert cache.stats()["misses"] == 0 and cache.stats()["hits"] == 0
    ids, _ = ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                           dev(ctx, x).device_ptr, yb.device_ptr)
    sel, _, want = capi.moe_layer(batch, hidden, width, experts, k, router, Q4_K, gu, Q6_K, dn, x)
    assert np.array_equal(ids, sel)
    got = yb.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
    for t in range(batch):
        assert_close(got[t], want[t], f"token {t}")
    cache.free()


def test_expert_cache_known_answer(ctx, golden):
    """src/expert.rs:266-325 through the HIP slots."""
    c = golden[0]["expert_lru"]
    lay = c["layout"]
    src = np.array(c["source"], dtype=np.uint8)
    cache = ExpertCache(ctx, src, [ExpertLayerLayout(**lay)], c["slots_per_layer"])
    assert cache.slots_per_layer() == 1
    for layer, expert, gate, down in c["accesses"]:
        def use(gate_up, down_buf):
            # the closure of src/expert.rs:290-298: gate.as_bytes(), down.as_bytes()
            assert gate_up.as_bytes().tolist() == gate
            assert down_buf.as_bytes().tolist() == down
        cache.with_expert(layer, expert, lambda: False, use)
    st = cache.stats()
    for key, value in c["expected_stats"].items():
        assert st[key] == value, key
    with pytest.raises(HipError) as e:
        cache.with_expert(0, 0, lambda: True, lambda *a: None)
    assert e.value.variant == "Cancelled"
    with pytest.raises(HipError) as e:
        cache.with_expert(0, 5, lambda: False, lambda *a: None)
    assert e.value.variant == "InvalidExpert"
    with pytest.raises(HipError) as e:
        cache.with_expert(3, 0, lambda: False, lambda *a: None)
    assert e.value.variant == "InvalidLayer"
    with pytest.raises(HipError) as e:
        ExpertCache(ctx, src, [ExpertLayerLayout(**lay)], 0)
    assert e.value.variant == "NoSlots"


def _expert_source(experts=16, hidden=2048, width=768, seed=4):
    gu_bytes = 2 * width * synth.row_bytes(Q4_K, hidden)
    dn_bytes = hidden * synth.row_bytes(Q6_K, width)
    gu = synth.quantized_matrix(Q4_K, experts * 2 * width, hidden, synth.weight_seed(seed, 0))
    dn = synth.quantized_matrix(Q6_K, experts * hidden, width, synth.weight_seed(seed, 1))
    # a 64-byte file header in front, so offsets are absolute file offsets
    blob = np.concatenate([np.full(64, 0x5A, np.uint8), gu, dn])
    layout = ExpertLayerLayout(experts, 64, gu_bytes, 64 + gu.size, dn_bytes)
    return blob, layout, gu, dn, gu_bytes, dn_bytes


def test_acquired_slots_feed_matvec_owned(ctx):
    """The drop-in path of src/gemma4/metal.rs:972-1031: with_expert hands the
    slot's gate_up and down buffers to a closure that runs matvec_owned on
    them (offset 0, the expert's byte length); the results match the oracle's
    matvec of that expert, and a range past the slot is MappedRange
    (src/metal.rs:1161-1168)."""
    hidden, width = 2048, 768
    blob, layout, gu, dn, gu_bytes, dn_bytes = _expert_source(hidden=hidden, width=width)
    cache = ExpertCache(ctx, blob, [layout], 2)
    x = synth.normal(synth.activation_seed(4, 77), hidden)
    for expert in (3, 11, 3):
        gu_e = gu[expert * gu_bytes:(expert + 1) * gu_bytes]
        dn_e = dn[expert * dn_bytes:(expert + 1) * dn_bytes]
        want_gu = capi.matvec(Q4_K, 2 * width, hidden, gu_e, x)
        act = synth.normal(synth.activation_seed(4, expert), width)
        want_dn = capi.matvec(Q6_K, hidden, width, dn_e, act)

        def closure(gate_up, down):
            assert len(gate_up) == gu_bytes and len(down) == dn_bytes
            out = np.zeros(2 * width, np.float32)
            ctx.matvec_owned(Q4_K, 2 * width, hidden, gate_up, 0, gu_bytes, x, out)
            out2 = np.zeros(hidden, np.float32)
            ctx.matvec_owned(Q6_K, hidden, width, down, 0, dn_bytes, act, out2)
            with pytest.raises(HipError) as e:
                ctx.matvec_owned(Q6_K, hidden // 2, width, down, dn_bytes // 2 + 630, dn_bytes // 2, act,
                                 np.zeros(hidden // 2, np.float32))
            assert e.value.variant == "MappedRange"
            assert e.value.detail == {"offset": dn_bytes // 2 + 630, "end": dn_bytes + 630, "length": dn_bytes}
            return out, out2

        got_gu, got_dn = cache.with_expert(0, expert, lambda: False, closure)
        assert_close(got_gu, want_gu, f"expert {expert} gate_up")
        assert_close(got_dn, want_dn, f"expert {expert} down")
    st = cache.stats()
    assert (st["hits"], st["misses"], st["evictions"]) == (1, 2, 0)
    cache.free()


def test_slot_reuse_waits_for_the_previous_expert_s_readers(ctx):
    """One slot.  Many GEMVs that read expert A's slot are enqueued (device
    entry points, nothing waits), then A is released and B acquired into the
    same slot: B's upload must wait for A's readers, so every A output still
    equals the oracle's, and B's bytes are B's."""
    hidden, width = 2048, 768
    blob, layout, gu, dn, gu_bytes, dn_bytes = _expert_source(hidden=hidden, width=width)
    cache = ExpertCache(ctx, blob, [layout], 1)
    x = synth.normal(synth.activation_seed(4, 88), hidden)
    xb = dev(ctx, x)
    reps = 64
    out = dev_out(ctx, reps * 2 * width * 4)
    slot, g, d = cache.acquire(0, 5)
    for r in range(reps):
        ctx.matvec_device(Q4_K, 2 * width, hidden, g.device_ptr, 1, xb.device_ptr, out.device_ptr + r * 2 * width * 4)
    cache.release(0, slot)
    slot2, g2, d2 = cache.acquire(0, 9)
    assert slot2 == slot and g2.device_ptr == g.device_ptr
    want_a = capi.matvec(Q4_K, 2 * width, hidden, gu[5 * gu_bytes:6 * gu_bytes], x)
    got = out.read(0, reps * 2 * width * 4, np.float32).reshape(reps, 2 * width)
    for r in range(reps):
        assert np.array_equal(got[r], got[0]), f"launch {r} read other bytes"
    assert_close(got[0], want_a, "expert A through its released slot")
    assert np.array_equal(g2.as_bytes(), gu[9 * gu_bytes:10 * gu_bytes])
    assert np.array_equal(d2.as_bytes(), dn[9 * dn_bytes:10 * dn_bytes])
    cache.release(0, slot2)
    cache.free()


def test_pinned_slots_are_never_evicted(ctx):
    """AllSlotsPinned when every slot of the layer is held; pins count (two
    acquires of one expert need two releases); releasing an unpinned slot is
    rejected."""
    blob, layout, gu, dn, gu_bytes, dn_bytes = _expert_source(experts=4, hidden=256, width=256)
    cache = ExpertCache(ctx, blob, [layout], 1)
    slot, g, _ = cache.acquire(0, 1)
    slot_again, _, _ = cache.acquire(0, 1)  # a hit on the pinned slot
    assert slot_again == slot
    with pytest.raises(HipError) as e:
        cache.acquire(0, 2)
    assert e.value.variant == "AllSlotsPinned" and e.value.detail == {"layer": 0}
    cache.release(0, slot)
    with pytest.raises(HipError) as e:
        cache.acquire(0, 2)  # still pinned once
    assert e.value.variant == "AllSlotsPinned"
    cache.release(0, slot)
    s2, g2, _ = cache.acquire(0, 2)
    assert np.array_equal(g2.as_bytes(), gu[2 * gu_bytes:3 * gu_bytes])
    cache.release(0, s2)
    with pytest.raises(HipError) as e:
        cache.release(0, s2)
    assert e.value.variant == "InvalidArgument"
    with pytest.raises(HipError) as e:
        cache.acquire(0, 4)
    assert e.value.variant == "InvalidExpert" and e.value.detail == {"layer": 0, "expert": 4, "count": 4}
    st = cache.stats()
    # src/expert.rs:166-229 counts: a miss (1), a hit, a refused miss, a refused
    # miss, a miss evicting 1; the refused misses count as misses with no read
    assert (st["hits"], st["misses"], st["evictions"], st["reads"]) == (1, 4, 1, 4)
    cache.free()


def test_file_backed_cache_matches_the_memory_backed_one(ctx, tmp_path):
    """ExpertCache over a file (the reference's Arc<File>, positional reads
    into pinned staging): C4 through moe_layer gives the same ids, outputs and
    LRU counters as the memory-backed cache; io_wait is the host's read time
    (positive); an expert past the end of the file fails with Io (unexpected
    end of file) and counts a miss but no read."""
    hidden, width, experts, k, batch = 2048, 768, 16, 4, 4
    blob, layout, gu, dn, gu_bytes, dn_bytes = _expert_source(experts=experts, hidden=hidden, width=width)
    path = tmp_path / "experts.bin"
    blob.tofile(path)
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(4, 5), experts * hidden) * np.float32(0.02))
    rb = dev(ctx, router)
    mem = ExpertCache(ctx, blob, [layout], 3)
    with open(path, "rb") as f:
        fil = ExpertCache.from_file(ctx, f, [layout], 3)
        ys = []
        for cache in (mem, fil):
            yb = dev_out(ctx, batch * hidden * 4)
            outs = []
            for step in range(3):
                x = synth.normal(synth.activation_seed(4, 300 + step), batch * hidden)
                ids, probs = ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                                           dev(ctx, x).device_ptr, yb.device_ptr)
                outs.append((ids, probs, yb.read(0, batch * hidden * 4, np.float32)))
            ys.append(outs)
        for (i1, p1, y1), (i2, p2, y2) in zip(*ys):
            assert np.array_equal(i1, i2) and np.array_equal(p1, p2)
            assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
        sm, sf = mem.stats(), fil.stats()
        for key in ("hits", "misses", "evictions", "reads", "bytes_read", "resident_bytes"):
            assert sm[key] == sf[key], key
        assert sf["io_wait_ns"] > 0 and sm["io_wait_ns"] > 0
        x = synth.normal(synth.activation_seed(4, 300), batch * hidden).reshape(batch, hidden)
        _, _, want = capi.moe_layer(batch, hidden, width, experts, k, router, Q4_K, gu, Q6_K, dn, x)
        for t in range(batch):
            assert_close(ys[1][0][2].reshape(batch, hidden)[t], want[t], f"file-backed token {t}")
        fil.free()
    # a layout that claims one more expert than the file holds
    short = ExpertLayerLayout(experts + 1, layout.gate_up_offset, gu_bytes, layout.down_offset, dn_bytes)
    with open(path, "rb") as f:
        cache = ExpertCache.from_file(ctx, f, [short], 2)
        with pytest.raises(HipError) as e:
            cache.acquire(0, experts)
        assert e.value.variant == "Io" and e.value.detail == {"os_error": 0}
        st = cache.stats()
        assert (st["misses"], st["reads"], st["bytes_read"]) == (1, 0, 0)
        slot, g, d = cache.acquire(0, 0)
        assert np.array_equal(g.as_bytes(), gu[:gu_bytes]) and np.array_equal(d.as_bytes(), dn[:dn_bytes])
        cache.release(0, slot)
        cache.free()
    mem.free()


def test_error_payloads_carry_the_variant_fields(ctx):
    """dmhip_last_error_detail: each validation variant carries the fields of
    its MetalError counterpart (src/metal.rs:3-126)."""
    x = np.zeros(256, np.float32)
    enc = np.zeros(144, np.uint8)
    out = np.zeros(1, np.float32)
    cases = [
        (lambda: ctx.matvec(Q4_K, 1, 256, enc, x[:10], out), "InvalidInputLength", {"expected": 256, "actual": 10}),
        (lambda: ctx.matvec(Q4_K, 1, 256, enc, x, np.zeros(2, np.float32)), "InvalidOutputLength",
         {"expected": 1, "actual": 2}),
        (lambda: ctx.matvec(13, 1, 256, np.zeros(176, np.uint8), x, out), "UnsupportedTensorType",
         {"kind": "Q5_K"}),
        (lambda: ctx.matvec(Q4_K, 1, 100, enc, x[:100], out), "InvalidElementCount",
         {"kind": "Q4_K", "elements": 100, "block_elements": 256}),
        (lambda: ctx.matvec(Q4_K, 1, 256, enc[:100], x, out), "InvalidByteLength",
         {"kind": "Q4_K", "expected": 144, "actual": 100}),
        (lambda: ctx.argmax([]), "EmptyInput", {"operation": "argmax"}),
        (lambda: ctx.argmax([1.0, np.inf]), "NonFinite", {"operation": "argmax"}),
        (lambda: ctx.top_k_softmax([1.0, 2.0], 3), "InvalidTopK", {"k": 3, "length": 2}),
        (lambda: ctx.rms_norm([1.0, 2.0], [1.0], 1e-6, np.zeros(2, np.float32)), "InvalidVectorLength",
         {"operation": "RMSNorm", "argument": "weight", "expected": 2, "actual": 1}),
        (lambda: ctx.rms_norm([1.0, 2.0], None, 0.0, np.zeros(2, np.float32)), "InvalidPositiveParameter",
         {"operation": "RMSNorm epsilon"}),
        (lambda: ctx.new_owned_buffer(0), "BufferAllocation", {"bytes": 0}),
    ]
    for fn, variant, detail in cases:
        with pytest.raises(HipError) as e:
            fn()
        assert e.value.variant == variant, (variant, e.value)
        assert e.value.detail == detail, (variant, e.value.detail)


@pytest.mark.parametrize("batch", [1, 4, 16])
def test_moe_layer_matches_oracle(ctx, batch):
    hidden, width, experts, k, slots = 2048, 768, 128, 8, 8
    print(f"C4 batch={batch}", flush=True)
    router, gu, dn, gu_bytes, dn_bytes = _moe_setup(hidden, width, experts)
    x = synth.normal(synth.activation_seed(4, batch), batch * hidden).reshape(batch, hidden)
    sel, wts, want = capi.moe_layer(batch, hidden, width, experts, k, router, Q4_K, gu, Q6_K, dn, x)
    src = PinnedHostBuffer(gu.size + dn.size)
    src.array[:gu.size] = gu
    src.array[gu.size:] = dn
    layout = ExpertLayerLayout(experts, 0, gu_bytes, gu.size, dn_bytes)
    cache = ExpertCache(ctx, src, [layout], slots)
    rb, xb, yb = dev(ctx, router), dev(ctx, x), dev_out(ctx, batch * hidden * 4)
    for step in range(2):  # second call runs on a warm cache
        ids, probs = ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                                   xb.device_ptr, yb.device_ptr)
        assert np.array_equal(ids, sel), "expert ids differ"
        assert np.allclose(probs, wts, rtol=1e-5, atol=1e-7)
        got = yb.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
        for t in range(batch):
            assert_close(got[t], want[t], f"C4 token {t} call {step}")
    # the cache decisions are the reference LRU's for the same acquire order
    lru = capi.Lru([experts], slots, gu_bytes, dn_bytes)
    for _ in range(2):
        for t in range(batch):
            for e in sel[t]:
                lru.acquire(0, int(e))
    st, ref = cache.stats(), lru.stats()
    for key in ("hits", "misses", "evictions", "reads", "bytes_read", "resident_bytes"):
        assert st[key] == ref[key], key
    cache.free()
    src.free()


@pytest.mark.parametrize("slots", [8, 16])
def test_moe_layer_resident_lookup_sequence(ctx, slots):
    """One-token MoE calls that take the device-side slot lookup once their
    experts are resident, and fall back when a slot is missing: tokens a, a,
    a, b, b, b, a, a, a non-finite token, a.  With 8 slots token b evicts
    token a's experts it does not share, so the later calls of a must not
    use a slot that now holds another expert.  Every clean call equals the
    oracle (ids, weights, output); the non-finite call returns NonFinite and
    acquires nothing; the cache counters equal the reference LRU's for the
    same acquire sequence."""
    hidden, width, experts, k = 2048, 768, 128, 8
    router, gu, dn, gu_bytes, dn_bytes = _moe_setup(hidden, width, experts)
    src = PinnedHostBuffer(gu.size + dn.size)
    src.array[:gu.size] = gu
    src.array[gu.size:] = dn
    cache = ExpertCache(ctx, src, [ExpertLayerLayout(experts, 0, gu_bytes, gu.size, dn_bytes)], slots)
    xs = {name: synth.normal(synth.activation_seed(45, i), hidden).reshape(1, hidden)
          for i, name in enumerate("ab")}
    want = {name: capi.moe_layer(1, hidden, width, experts, k, router, Q4_K, gu, Q6_K, dn, x)
            for name, x in xs.items()}
    bad = xs["a"].copy()
    bad[0, 100] = np.nan
    rb, yb = dev(ctx, router), dev_out(ctx, hidden * 4)
    dx = {name: dev(ctx, x) for name, x in xs.items()}
    lru = capi.Lru([experts], slots, gu_bytes, dn_bytes)
    first = {}
    for step, name in enumerate(["a", "a", "a", "b", "b", "b", "a", "a", "bad", "a"]):
        print(f"slots={slots} call {step}: token {name}", flush=True)
        if name == "bad":
            before = cache.stats()
            with pytest.raises(HipError) as e:
                ctx.moe_layer(cache, 0, 1, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                              dev(ctx, bad).device_ptr, yb.device_ptr)
            assert e.value.variant == "NonFinite"
            after = cache.stats()
            assert (after["hits"], after["misses"]) == (before["hits"], before["misses"])
            continue
        sel, wts, out = want[name]
        ids, probs = ctx.moe_layer(cache, 0, 1, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                                   dx[name].device_ptr, yb.device_ptr)
        assert np.array_equal(ids, sel), f"call {step}: expert ids differ"
        assert np.allclose(probs, wts, rtol=1e-5, atol=1e-7)
        got = yb.read(0, hidden * 4, np.float32)
        assert_close(got, out[0], f"call {step} token {name}")
        # the host path (first call of a token) and the device lookup with the
        # combine fused into the down launch (later calls) agree bit for bit
        first.setdefault(name, got.copy())
        assert np.array_equal(bits(got), bits(first[name])), f"call {step}: output differs from the token's first call"
        for e_id in sel[0]:
            lru.acquire(0, int(e_id))
    st, ref = cache.stats(), lru.stats()
    for key in ("hits", "misses", "evictions", "reads", "bytes_read", "resident_bytes"):
        assert st[key] == ref[key], key
    cache.free()
    src.free()


@pytest.mark.parametrize("batch,slots", [(2, 24), (4, 128), (8, 128)])
def test_moe_layer_resident_lookup_batches(ctx, batch, slots):
    """Batches of 2-8 tokens take the device-side slot lookup once every
    selected expert is resident (one job per token and selection, the
    combine per token fused into the down launch or run behind it), and the
    host path when a
    slot is missing: batches a, a, a, b, b, a, a, a non-finite batch, a.
    With 24 slots and 2 tokens, batch b evicts some of a's experts, so the
    later calls of a find a slot missing at least once.  Every clean call
    equals the oracle (ids, weights, output); calls of one batch on the
    lookup path agree bit for bit; the cache counters equal the reference
    LRU's for the same acquire sequence."""
    hidden, width, experts, k = 2048, 256, 128, 8
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(51, 0), experts * hidden) * np.float32(0.02))
    gu_bytes, dn_bytes = 2 * width * synth.row_bytes(Q4_K, hidden), hidden * synth.row_bytes(Q6_K, width)
    gu = synth.quantized_matrix(Q4_K, experts * 2 * width, hidden, synth.weight_seed(51, 1))
    dn = synth.quantized_matrix(Q6_K, experts * hidden, width, synth.weight_seed(51, 2))
    src = PinnedHostBuffer(gu.size + dn.size)
    src.array[:gu.size] = gu
    src.array[gu.size:] = dn
    cache = ExpertCache(ctx, src, [ExpertLayerLayout(experts, 0, gu_bytes, gu.size, dn_bytes)], slots)
    xs = {name: synth.normal(synth.activation_seed(51, 10 * batch + i), batch * hidden).reshape(batch, hidden)
          for i, name in enumerate("ab")}
    want = {name: capi.moe_layer(batch, hidden, width, experts, k, router, Q4_K, gu, Q6_K, dn, x)
            for name, x in xs.items()}
    bad = xs["a"].copy()
    bad[batch - 1, 7] = np.inf
    rb, yb = dev(ctx, router), dev_out(ctx, batch * hidden * 4)
    dx = {name: dev(ctx, x) for name, x in xs.items()}
    lru = capi.Lru([experts], slots, gu_bytes, dn_bytes)
    seen = {}
    try_lookup = True  # the layer's state: a lookup is tried after a call whose experts were all resident
    paths = []
    for step, name in enumerate(["a", "a", "a", "b", "b", "a", "a", "bad", "a"]):
        print(f"batch={batch} slots={slots} call {step}: {name}", flush=True)
        if name == "bad":
            before = cache.stats()
            with pytest.raises(HipError) as e:
                ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                              dev(ctx, bad).device_ptr, yb.device_ptr)
            assert e.value.variant == "NonFinite"
            after = cache.stats()
            assert (after["hits"], after["misses"]) == (before["hits"], before["misses"])
            continue
        sel, wts, out = want[name]
        misses = cache.stats()["misses"]
        ids, probs = ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                                   dx[name].device_ptr, yb.device_ptr)
        assert np.array_equal(ids, sel), f"call {step}: expert ids differ"
        assert np.allclose(probs, wts, rtol=1e-5, atol=1e-7)
        got = yb.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
        for t in range(batch):
            assert_close(got[t], out[t], f"call {step} batch {name} token {t}")
        hits_only = cache.stats()["misses"] == misses
        path = "lookup" if try_lookup and hits_only else "host"
        try_lookup = hits_only
        paths.append(path)
        # each path repeats its results bit for bit
        if (name, path) in seen:
            assert np.array_equal(bits(got), bits(seen[name, path])), f"call {step}: output differs"
        seen.setdefault((name, path), got.copy())
        for t in range(batch):
            for e_id in sel[t]:
                lru.acquire(0, int(e_id))
    st, ref = cache.stats(), lru.stats()
    for key in ("hits", "misses", "evictions", "reads", "bytes_read", "resident_bytes"):
        assert st[key] == ref[key], key
    assert "lookup" in paths, paths
    cache.free()
    src.free()


def test_moe_layer_lookup_wide_router(ctx):
    """Two tokens over a router wider than 8192 columns (the exact fold's
    expert-parallel kernel, which writes the device-side lookup itself):
    four calls of one batch, the host path until the experts are resident,
    then the lookup; every call equals the oracle and each path repeats its
    results bit for bit."""
    hidden, width, experts, k, batch, slots = 8448, 256, 32, 4, 2, 32
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(52, 0), experts * hidden) * np.float32(0.02))
    gu_bytes, dn_bytes = 2 * width * synth.row_bytes(Q4_K, hidden), hidden * synth.row_bytes(Q6_K, width)
    gu = synth.quantized_matrix(Q4_K, experts * 2 * width, hidden, synth.weight_seed(52, 1))
    dn = synth.quantized_matrix(Q6_K, experts * hidden, width, synth.weight_seed(52, 2))
    cache = ExpertCache(ctx, np.concatenate([gu, dn]), [ExpertLayerLayout(experts, 0, gu_bytes, gu.size, dn_bytes)],
                        slots)
    x = synth.normal(synth.activation_seed(52, 0), batch * hidden).reshape(batch, hidden)
    sel, wts, want = capi.moe_layer(batch, hidden, width, experts, k, router, Q4_K, gu, Q6_K, dn, x)
    rb, xb, yb = dev(ctx, router), dev(ctx, x), dev_out(ctx, batch * hidden * 4)
    seen, try_lookup, paths = {}, True, []
    for step in range(4):
        misses = cache.stats()["misses"]
        ids, probs = ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                                   xb.device_ptr, yb.device_ptr)
        assert np.array_equal(ids, sel), f"call {step}: expert ids differ"
        assert np.allclose(probs, wts, rtol=1e-5, atol=1e-7)
        got = yb.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
        for t in range(batch):
            assert_close(got[t], want[t], f"call {step} token {t}")
        hits_only = cache.stats()["misses"] == misses
        path = "lookup" if try_lookup and hits_only else "host"
        try_lookup = hits_only
        paths.append(path)
        if path in seen:
            assert np.array_equal(bits(got), bits(seen[path])), f"call {step}: output differs"
        seen.setdefault(path, got.copy())
    print("paths", paths, flush=True)
    assert "lookup" in paths, paths
    cache.free()


# ---- the MoE layer's certified router: planted near-ties ------------------------

def _moe_run_planted(ctx, router, x, hidden, width, experts, k, seed):
    """One MoE layer call per token batch, twice (a cache with a slot per
    expert: the second call of one token takes the device lookup), against
    the oracle: ids exact and in order, weights within 1e-5, output within the
    GEMV tolerance.  Returns the oracle's ids."""
    batch = x.shape[0]
    gu_bytes, dn_bytes = 2 * width * synth.row_bytes(Q4_K, hidden), hidden * synth.row_bytes(Q6_K, width)
    gu = synth.quantized_matrix(Q4_K, experts * 2 * width, hidden, synth.weight_seed(seed, 1))
    dn = synth.quantized_matrix(Q6_K, experts * hidden, width, synth.weight_seed(seed, 2))
    cache = ExpertCache(ctx, np.concatenate([gu, dn]), [ExpertLayerLayout(experts, 0, gu_bytes, gu.size, dn_bytes)],
                        experts)
    sel, wts, want = capi.moe_layer(batch, hidden, width, experts, k, router, Q4_K, gu, Q6_K, dn, x)
    rb, xb, yb = dev(ctx, router), dev(ctx, x), dev_out(ctx, batch * hidden * 4)
    for step in range(2):
        ids, probs = ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                                   xb.device_ptr, yb.device_ptr)
        assert np.array_equal(ids, sel), f"call {step}: expert ids differ: {ids.tolist()} != {sel.tolist()}"
        assert np.allclose(probs, wts, rtol=1e-5, atol=1e-7)
        got = yb.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
        for t in range(batch):
            assert_close(got[t], want[t], f"call {step} token {t}")
    cache.free()
    return sel


def test_moe_router_planted_near_ties(ctx):
    """Rows whose order under the reference's sequential f32 fold is the
    reverse of their exact order, and two identical rows (an exact tie: the
    lower index first), among the top k.  The certified router cannot order
    either pair from its bounds and folds them exactly: the ids and their
    order are the reference's (src/cpu.rs:232-260)."""
    hidden, width, experts, k = 2048, 256, 128, 8
    rng = np.random.default_rng(4601)
    x = rng.standard_normal((3, hidden)).astype(np.float32)
    # a and c lean towards every token, so their logits lead every selection
    lean = x.sum(0)
    a = synth.to_bf16_bits(np.float32(0.03) * lean + np.float32(0.01) * rng.standard_normal(hidden).astype(np.float32))
    # b = a with weight i0 one bf16 step larger and weight j m steps away,
    # so that exact(b) - exact(a) = delta (exact in double) is a fraction of
    # an f32 ulp of the logit: find such a b whose fold over token 0 orders
    # it against a the other way (a single changed weight cannot: rounding is
    # monotone, so the two folds keep the order of their sums)
    f64 = lambda v: synth.bf16_bits_to_f32(np.asarray(v, np.uint16)).astype(np.float64)
    wa, x0 = f64(a), x[0].astype(np.float64)
    fa = capi.matvec_bf16(1, hidden, a, x[0])[0]
    b, delta = None, 0.0
    for i0 in range(8):
        d0 = (f64(a[i0] + np.uint16(1)) - wa[i0]) * x0[i0]
        rows, deltas = [], []
        for m in [v for v in range(-12, 13) if v]:
            bj = (a.astype(np.int64) + m).astype(np.uint16)
            dt = d0 + (f64(bj) - wa) * x0
            ok = (np.sign(f64(bj)) == np.sign(wa)) & (np.arange(hidden) > 8) & (np.abs(dt) < 1.5e-6) & (dt != 0)
            for j in np.nonzero(ok)[0]:
                r = a.copy()
                r[i0] += np.uint16(1)
                r[j] = bj[j]
                rows.append(r)
                deltas.append(dt[j])
        fb = capi.matvec_bf16(len(rows), hidden, np.stack(rows), x[0])
        for r, d, fv in zip(rows, deltas, fb):
            if (d > 0 and fv < fa) or (d < 0 and fv > fa):
                b, delta = r, d
                break
        if b is not None:
            break
    assert b is not None, "no planted pair reverses the fold order"
    router = synth.to_bf16_bits(rng.standard_normal((experts, hidden)).astype(np.float32) * np.float32(0.02))
    router[17] = a
    router[40] = b
    c = synth.to_bf16_bits(np.float32(0.02) * lean + np.float32(0.01) * rng.standard_normal(hidden).astype(np.float32))
    router[5] = c
    router[90] = c
    sel = _moe_run_planted(ctx, router.reshape(-1), x, hidden, width, experts, k, 46)
    s0 = sel[0].tolist()
    assert 17 in s0 and 40 in s0 and 5 in s0 and 90 in s0, s0
    # the planted reversal: the reference orders the pair by its fold, not by
    # the exact sums
    exact_first = 40 if delta > 0 else 17
    assert s0.index(exact_first) > s0.index(57 - exact_first), s0
    for t in range(3):
        assert sel[t].tolist().index(5) < sel[t].tolist().index(90)


@pytest.mark.parametrize("hidden,experts,k,tokens", [(2048, 128, 8, 2), (6144, 32, 4, 2), (2048, 128, 8, 12)])
def test_moe_router_all_rows_equal(ctx, hidden, experts, k, tokens):
    """Every router row the same: every logit ties, and the reference selects
    rows 0 .. k - 1 in index order with equal weights; the certified router
    folds every row exactly (two rows per LDS batch up to 4096 columns, one
    above).  Up to 8 tokens its workgroups have 4 waves, above 8."""
    width = 256
    rng = np.random.default_rng(4602)
    row = synth.to_bf16_bits(rng.standard_normal(hidden).astype(np.float32) * np.float32(0.02))
    router = np.tile(row, experts)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    sel = _moe_run_planted(ctx, router, x, hidden, width, experts, k, 47)
    assert sel.tolist() == [list(range(k))] * tokens


@pytest.mark.parametrize("scale", [0.02, 3e-18])
def test_moe_router_random_tokens(ctx, scale):
    """64 random tokens (4 calls of 16) through the certified router: every
    call's ids, in order, are the oracle's sequential fold's; at this data
    about one token in fifty needs the exact fold of its near-tied rows.  The
    tiny scale puts the logits near 1e-16, far from the unit scale."""
    hidden, width, experts, k, batch = 2048, 256, 128, 8, 16
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(50, 0), experts * hidden) * np.float32(scale))
    for call in range(4):
        x = synth.normal(synth.activation_seed(50, call), batch * hidden).reshape(batch, hidden)
        print(f"scale={scale} call {call}", flush=True)
        _moe_run_planted(ctx, router, x, hidden, width, experts, k, 50)


@pytest.mark.parametrize("tokens", [3, 10])
def test_moe_router_odd_shapes(ctx, tokens):
    """The certified router over a partial last round of columns (hidden 2816:
    352 pieces of 8) and a partial last workgroup (202 experts), with 4-wave
    (3 tokens) and 8-wave (10 tokens) workgroups."""
    hidden, width, experts, k = 2816, 256, 202, 6
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(48, 0), experts * hidden) * np.float32(0.02))
    x = synth.normal(synth.activation_seed(48, 1), tokens * hidden).reshape(tokens, hidden)
    _moe_run_planted(ctx, router, x, hidden, width, experts, k, 48)


def test_moe_router_fold_overflow_is_non_finite(ctx):
    """A row whose sequential f32 fold overflows (partial sums past FLT_MAX)
    although its exact sum is 0: the reference's logit is infinite and
    top_k_softmax rejects it (src/cpu.rs:240-245), so the layer returns
    NonFinite and acquires nothing."""
    hidden, width, experts, k = 2048, 256, 128, 8
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(49, 0), experts * hidden) * np.float32(0.02))
    router = router.reshape(experts, hidden)
    router[3, :hidden // 2] = synth.to_bf16_bits(np.ones(hidden // 2, np.float32))
    router[3, hidden // 2:] = synth.to_bf16_bits(-np.ones(hidden // 2, np.float32))
    x = np.full((1, hidden), 1e36, dtype=np.float32)
    assert np.isinf(capi.matvec_bf16(experts, hidden, router, x[0])[3])
    gu_bytes, dn_bytes = 2 * width * synth.row_bytes(Q4_K, hidden), hidden * synth.row_bytes(Q6_K, width)
    gu = synth.quantized_matrix(Q4_K, experts * 2 * width, hidden, synth.weight_seed(49, 1))
    dn = synth.quantized_matrix(Q6_K, experts * hidden, width, synth.weight_seed(49, 2))
    cache = ExpertCache(ctx, np.concatenate([gu, dn]), [ExpertLayerLayout(experts, 0, gu_bytes, gu.size, dn_bytes)],
                        experts)
    rb, xb, yb = dev(ctx, router.reshape(-1)), dev(ctx, x), dev_out(ctx, hidden * 4)
    with pytest.raises(HipError) as e:
        ctx.moe_layer(cache, 0, 1, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K, xb.device_ptr,
                      yb.device_ptr)
    assert e.value.variant == "NonFinite"
    assert cache.stats()["misses"] == 0 and cache.stats()["hits"] == 0
    cache.free()


# ---- config 5: prefill GEMM ----------------------------------------------------

def _gemm_check(ctx, kind, m, n, k, seed, what):
    """dmhip_gemm_device against the oracle's one-matvec-per-token GEMM
    (src/gemma4/metal.rs:514-536 over src/cpu.rs:345-399), every token."""
    print(f"{what}: type {kind} m={m} n={n} k={k}", flush=True)
    a = synth.to_bf16_bits(synth.normal(synth.activation_seed(seed, kind), m * k))
    w = synth.quantized_matrix(kind, n, k, synth.weight_seed(seed, n * 31 + kind))
    want = capi.gemm_tokenwise(kind, m, n, k, a, w)
    ab, wb, cb = dev(ctx, a), dev(ctx, w), dev_out(ctx, m * n * 4)
    ws = dev_out(ctx, ctx.gemm_workspace_bytes(m, k))
    ctx.gemm_device(kind, m, n, k, ab.device_ptr, wb.device_ptr, cb.device_ptr, ws.device_ptr, len(ws))
    got = cb.read(0, m * n * 4, np.float32).reshape(m, n)
    worst = 0.0
    for r in range(m):
        e, _ = assert_close(got[r], want[r], f"{what} type {kind} token {r}")
        worst = max(worst, e)
    exact, scale = exact_products(kind, n, k, w, synth.bf16_bits_to_f32(a).reshape(m, k))
    ch = assert_channel_close(got, exact, scale, CHANNEL_TOL_GEMM, f"{what} type {kind}")
    print(f"  worst rel_err={worst:.2e} channel={ch:.2e} (oracle {channel_err(want, exact, scale):.2e})",
          flush=True)
    return worst


@pytest.mark.parametrize("n", [4096, 12288])
def test_prefill_gemm_matches_oracle(ctx, n):
    """C5: Q4_K, 512 tokens, K = 4096; every token of both N (all 4 M tiles,
    every N tile and XCD position)."""
    _gemm_check(ctx, Q4_K, 512, n, 4096, 5, "C5")


@pytest.mark.parametrize("kind", [Q6_K, Q8_0])
@pytest.mark.parametrize("n,k", [(4096, 4096), (4096, 12288)])
def test_prefill_gemm_q6_k_and_q8_0_on_mfma(ctx, kind, n, k):
    """The MFMA GEMM for the other two quantized types of the north star, at
    M = 512 and K = 4096 / 12288 (src/cpu.rs:576-583, :618-645)."""
    _gemm_check(ctx, kind, 512, n, k, 6, "prefill")


@pytest.mark.parametrize("kind", [Q4_K, Q6_K, Q8_0])
@pytest.mark.parametrize("m,n,k", [(17, 64, 256), (100, 200, 2048), (65, 264, 2816), (300, 136, 4608)])
def test_prefill_gemm_ragged_shapes(ctx, kind, m, n, k):
    """M not a multiple of the 128-row tile (padding rows; 17 = the smallest
    MFMA prefill), N not a multiple of the 64-column tile, a single K block
    (three waves without blocks), and K quarters of unequal length; K = 2816
    (11 blocks) gives Q6_K rows whose 210-byte blocks start 2 bytes off a
    dword boundary on every other row."""
    _gemm_check(ctx, kind, m, n, k, 7, "ragged")


def test_objects_outliving_their_context_exit_cleanly():
    """Regression: device buffers and caches freed after their context was
    closed (the order Python's collector may pick at exit)."""
    import subprocess
    import sys
    code = (
        "import numpy as np\n"
        "from diskmule_amd import HipContext, ExpertCache, ExpertLayerLayout\n"
        "ctx = HipContext(0)\n"
        "a = ctx.device_array(np.arange(1000, dtype=np.float32))\n"
        "m = ctx.map_read_only(np.zeros(4096, np.uint8))\n"
        "c = ExpertCache(ctx, np.arange(16, dtype=np.uint8), [ExpertLayerLayout(2, 0, 4, 8, 4)], 1)\n"
        "ctx.close()\n"
        "del a, m, c\n"
        "print('clean')\n"
    )
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120,
                       cwd=__import__("os").path.dirname(__import__("os").path.dirname(__file__)))
    assert r.returncode == 0 and "clean" in r.stdout, (r.returncode, r.stderr[-2000:])
