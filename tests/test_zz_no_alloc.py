"""bh_attn_decode_noalloc (attention without any device allocation: split scratch in a fixed
per-device array) against bh_attn_decode, through the C ABI: two calls in a row, the second
with a smaller input, each equal bit for bit to the allocating entry point's output (same
kernels, same split plan); a plan larger than the fixed scratch is refused."""
import numpy as np
import pytest

from bramha_amd import ops
from bramha_amd._lib import BhError, check, lib

pytestmark = pytest.mark.gpu


def _inputs(plane, B, T, seed, nq=14, nkv=2, hd=64):
    D = lambda a: ops.DeviceArray.from_numpy(plane, a)  # noqa: E731
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((nkv, B * T, hd)).astype(np.float16)
    v = rng.standard_normal((nkv, B * T, hd)).astype(np.float16)
    kp, vp = ops.pack_kv_f16(k, v)
    q = rng.standard_normal((B, nq * hd)).astype(np.float32)
    return [D(q), D(kp), D(vp), D((np.arange(B) * T).astype(np.int64)), D(np.full(B, T, np.int32))]


def _noalloc(plane, ins, B, T, nq=14, nkv=2, hd=64):
    q, k, v, off, ln = ins
    out = ops.DeviceArray(plane, (B, nq * hd), np.float32)
    check(lib.bh_attn_decode_noalloc(plane.ctx, q.ptr, k.ptr, v.ptr, 1, B * T, off.ptr, ln.ptr, B, nq, nkv, hd, T,
                                     out.ptr, None), plane.ctx)
    return out.numpy()


@pytest.mark.parametrize("shape", [(8, 4096, 2, 2048), (1, 32768, 1, 8192)])
def test_noalloc_attention_matches_allocating_entry_point(plane, shape):
    B1, T1, B2, T2 = shape  # the second call is smaller (fewer rows, fewer splits)
    for i, (B, T) in enumerate(((B1, T1), (B2, T2))):
        ins = _inputs(plane, B, T, seed=90 + 10 * i + B)
        want = ops.attn_decode(plane, *ins, 14, 2, 64, T).numpy()
        got = _noalloc(plane, ins, B, T)
        assert np.isfinite(got).all()
        assert np.array_equal(got, want), (B, T)
        got2 = _noalloc(plane, ins, B, T)  # the counters were left at zero by the first call
        assert np.array_equal(got2, want), (B, T)


def test_noalloc_refuses_plans_beyond_its_scratch(plane):
    """255 rows of 8 query heads on one KV head of 128 dims over 2048 rows split in 2: partials of
    255 * 8 * 2 * 130 * 4 = 2121600 bytes, above the 2 MiB of the fixed scratch. Refused on the
    host (no kernel runs); the allocating entry point runs the same call."""
    B, T, nq, nkv, hd = 255, 2048, 8, 1, 128
    D = lambda a: ops.DeviceArray.from_numpy(plane, a)  # noqa: E731
    q = D(np.zeros((B, nq * hd), np.float32))
    k = D(np.zeros((nkv, 2048 * hd), np.float16))
    off = D(np.zeros(B, np.int64))
    ln = D(np.full(B, T, np.int32))
    out = ops.DeviceArray(plane, (B, nq * hd), np.float32)
    with pytest.raises(BhError) as e:
        check(lib.bh_attn_decode_noalloc(plane.ctx, q.ptr, k.ptr, k.ptr, 1, 2048, off.ptr, ln.ptr, B, nq, nkv, hd, T,
                                         out.ptr, None), plane.ctx)
    assert e.value.status == -8  # BH_ERR_CAPACITY
    check(lib.bh_attn_decode(plane.ctx, q.ptr, k.ptr, k.ptr, 1, 2048, off.ptr, ln.ptr, B, nq, nkv, hd, T, out.ptr,
                             None), plane.ctx)
    assert np.array_equal(out.numpy(), np.zeros((B, nq * hd), np.float32))
