"""The allocation-free FFN entry point (dmhip_ffn_device_noalloc) against the
workspace entry point it mirrors (dmhip_ffn_device): same kernels on the same
inputs, so the outputs must be identical bit for bit; two calls in a row, the
second smaller; a shape beyond the fixed scratch is rejected; and the call
allocates no device memory."""
import ctypes

import numpy as np
import pytest

from diskmule_amd import HipContext, HipError, synth
from oracle import capi
from tests.tolerance import assert_close

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 12, 14


def _free_device_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def _weights(hidden, ffn, seed):
    g = synth.quantized_matrix(Q4_K, ffn, hidden, synth.weight_seed(seed, 0))
    u = synth.quantized_matrix(Q4_K, ffn, hidden, synth.weight_seed(seed, 1))
    d = synth.quantized_matrix(Q6_K, hidden, ffn, synth.weight_seed(seed, 2))
    return g, u, d


def test_noalloc_ffn_matches_the_workspace_entry_point():
    ctx = HipContext(0)
    try:
        calls = [(8, 4096, 12288, 3), (2, 2048, 1536, 9)]  # the second call is smaller
        prepared = []
        for batch, hidden, ffn, seed in calls:
            g, u, d = _weights(hidden, ffn, seed)
            h = synth.normal(synth.activation_seed(seed, batch), batch * hidden).reshape(batch, hidden)
            bufs = [ctx.device_array(a) for a in (g, u, d, h)]
            prepared.append((batch, hidden, ffn, g, u, d, h, bufs, ctx.new_owned_buffer(batch * hidden * 4)))
        ctx.synchronize()
        free_before = _free_device_bytes()
        for batch, hidden, ffn, g, u, d, h, (gb, ub, db, hb), yb in prepared:
            print(f"noalloc FFN batch={batch} hidden={hidden} ffn={ffn}", flush=True)
            ctx.ffn_device_noalloc(batch, hidden, ffn, Q4_K, gb.device_ptr, Q4_K, ub.device_ptr, Q6_K, db.device_ptr,
                                   1e-6, hb.device_ptr, yb.device_ptr)
        ctx.synchronize()
        assert _free_device_bytes() == free_before, "the allocation-free call allocated device memory"
        for batch, hidden, ffn, g, u, d, h, (gb, ub, db, hb), yb in prepared:
            got = yb.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
            ws = ctx.new_owned_buffer(ctx.ffn_workspace_bytes(batch, hidden, ffn))
            yw = ctx.new_owned_buffer(batch * hidden * 4)
            ctx.ffn_device(batch, hidden, ffn, Q4_K, gb.device_ptr, Q4_K, ub.device_ptr, Q6_K, db.device_ptr,
                           1e-6, hb.device_ptr, yw.device_ptr, ws.device_ptr, len(ws))
            want = yw.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"batch {batch}"
            ref = capi.dense_ffn(batch, hidden, ffn, Q4_K, g, Q4_K, u, Q6_K, d, h)
            for b in range(batch):
                assert_close(got[b], ref[b], f"batch {batch} token {b}")
        # beyond the fixed scratch: rejected before any work
        big_h, big_f = 32768, 65536
        assert ctx.ffn_workspace_bytes(16, big_h, big_f) > ctx.ffn_noalloc_scratch_bytes()
        gb, ub, db, hb, yb = prepared[0][7] + [prepared[0][8]]
        with pytest.raises(HipError) as e:
            ctx.ffn_device_noalloc(16, big_h, big_f, Q4_K, gb.device_ptr, Q4_K, ub.device_ptr, Q6_K, db.device_ptr,
                                   1e-6, hb.device_ptr, yb.device_ptr)
        assert e.value.variant == "InvalidArgument"
    finally:
        ctx.close()


def test_noalloc_ffn_with_mixed_gate_and_up_types():
    """An unfused FFN whose gate is Q6_K and up Q4_K at batch 8: the up
    matrix's activation fragments (nine scale slots per block) are larger
    than the gate's (eight) and the down input's, and the lent region is
    sized for the largest, so the call completes and equals the workspace
    entry point bit for bit."""
    ctx = HipContext(0)
    try:
        batch, hidden, ffn, seed = 8, 4096, 1024, 21
        g = synth.quantized_matrix(Q6_K, ffn, hidden, synth.weight_seed(seed, 0))
        u = synth.quantized_matrix(Q4_K, ffn, hidden, synth.weight_seed(seed, 1))
        d = synth.quantized_matrix(Q6_K, hidden, ffn, synth.weight_seed(seed, 2))
        h = synth.normal(synth.activation_seed(seed, batch), batch * hidden).reshape(batch, hidden)
        gb, ub, db, hb = (ctx.device_array(a) for a in (g, u, d, h))
        yb, yw = ctx.new_owned_buffer(batch * hidden * 4), ctx.new_owned_buffer(batch * hidden * 4)
        ws = ctx.new_owned_buffer(ctx.ffn_workspace_bytes(batch, hidden, ffn))
        print(f"noalloc FFN mixed types batch={batch} hidden={hidden} ffn={ffn}", flush=True)
        ctx.ffn_device_noalloc(batch, hidden, ffn, Q6_K, gb.device_ptr, Q4_K, ub.device_ptr, Q6_K, db.device_ptr,
                               1e-6, hb.device_ptr, yb.device_ptr)
        ctx.ffn_device(batch, hidden, ffn, Q6_K, gb.device_ptr, Q4_K, ub.device_ptr, Q6_K, db.device_ptr,
                       1e-6, hb.device_ptr, yw.device_ptr, ws.device_ptr, len(ws))
        got = yb.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
        want = yw.read(0, batch * hidden * 4, np.float32).reshape(batch, hidden)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        ref = capi.dense_ffn(batch, hidden, ffn, Q6_K, g, Q4_K, u, Q6_K, d, h)
        for b in range(batch):
            assert_close(got[b], ref[b], f"mixed types token {b}")
    finally:
        ctx.close()
