"""GPU parity of the single operators against the oracle (and float64 where the oracle
is itself float32). Tolerances are stated per test."""
import numpy as np
import pytest

import oracle
import ref64
from bramha_amd import _lib, ops
from bramha_amd._lib import BH_F32, BH_Q4_G32, BH_Q4_ROW, BH_Q8_ROW, BhError
from bramha_amd.plane import try_gpu_matvec

pytestmark = pytest.mark.gpu

QWEN_SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864), (151936, 896)]  # (N, K)


def _quant(fmt, w):
    if fmt == BH_F32:
        return w, None, w
    if fmt == BH_Q8_ROW:
        q, s = oracle.quantize_int8(w)
        return q, s, oracle.dequantize_int8(q, s)
    if fmt == BH_Q4_ROW:
        q, s = oracle.quantize_int4(w)
        return q, s, oracle.dequantize_int4(q, s, w.shape[1])
    q, s = oracle.quantize_q4g32(w)
    return q, s, oracle.dequantize_q4g32(q, s, w.shape[1])


def _w(seed, n, k, sigma=0.02):
    return (np.random.default_rng(seed).standard_normal((n, k)) * sigma).astype(np.float32)


@pytest.mark.parametrize("fmt", [BH_F32, BH_Q8_ROW, BH_Q4_ROW, BH_Q4_G32])
@pytest.mark.parametrize("n,k", [(64, 128), (37, 96), (896, 896), (4864, 896), (896, 4864)])
def test_dequant_bit_exact(plane, fmt, n, k):
    w = _w(n + k, n, k)
    w[0] = 0
    q, s, deq = _quant(fmt, w)
    dw = ops.DeviceWeight(plane, fmt, n, k, q, s)
    got = dw.dequant().numpy()
    assert np.array_equal(got.view(np.uint32), deq.view(np.uint32))


def test_dequant_bit_exact_lm_head(plane):
    w = _w(9, 151936, 896)
    q, s, deq = _quant(BH_Q4_G32, w)
    got = ops.DeviceWeight(plane, BH_Q4_G32, 151936, 896, q, s).dequant().numpy()
    assert np.array_equal(got.view(np.uint32), deq.view(np.uint32))


def _check_gemv(y, deq, x):
    """Within f32 accumulation error of the exact product: |y - y64| <= 2e-6 * (|W| |x|) + 1e-7."""
    want = x.astype(np.float64) @ deq.astype(np.float64).T
    bound = 2e-6 * (np.abs(x).astype(np.float64) @ np.abs(deq).astype(np.float64).T) + 1e-7
    err = np.abs(y - want)
    assert np.all(err <= bound), float((err / bound).max())


_QCACHE = {}


def _q4_cached(n, k):
    if (n, k) not in _QCACHE:
        _QCACHE.clear()
        _QCACHE[(n, k)] = _quant(BH_Q4_G32, _w(n * 7 + k, n, k))
    return _QCACHE[(n, k)]


@pytest.mark.parametrize("n,k", QWEN_SHAPES)
@pytest.mark.parametrize("batch", [1, 4, 16, 32])
def test_gemv_q4g32_qwen_shapes(plane, n, k, batch):
    q, s, deq = _q4_cached(n, k)
    x = np.random.default_rng(batch).standard_normal((batch, k)).astype(np.float32)
    dw = ops.DeviceWeight(plane, BH_Q4_G32, n, k, q, s)
    y = dw.gemv(ops.DeviceArray.from_numpy(plane, x)).numpy()
    _check_gemv(y, deq, x)
    if batch == 1:  # the reference GEMV over the dequantized weights
        yo = oracle.matvec_mul_into(oracle.F32, x[0], deq, None, n)
        assert np.max(np.abs(y[0] - yo)) <= 1e-5 * max(1.0, np.abs(yo).max())


def _limb_edge_rows(k):
    """Activation rows that stress the batch-1 group-32 pass, whose activations are turned into
    8 signed 4-bit limbs under one exponent per 32-element chunk: huge and tiny values in one
    chunk, outliers 1e4 above their chunk, all-zero chunks, a chunk below the 2^-97 cut, powers
    of two at the chunk maximum, negative maxima, subnormals, and magnitudes near the f32 limit."""
    rng = np.random.default_rng(7)
    rows = []
    x = rng.standard_normal(k).astype(np.float32)
    x[0], x[1], x[2] = 1e30, -1e-30, 3e-8
    x[32:64] = 0.0
    x[64:96] = 1e-35 * rng.standard_normal(32)
    rows.append(x)
    x = rng.standard_normal(k).astype(np.float32)
    x[3::32] = 1e4 * np.sign(x[3::32])
    rows.append(x)
    x = np.zeros(k, np.float32)
    x[::32] = 2.0 ** np.arange(-60, -60 + k // 32)[: len(x[::32])]   # maxima at powers of two
    x[5::32] = -x[::32] * 0.75
    rows.append(x)
    x = -np.abs(rng.standard_normal(k)).astype(np.float32)            # negative maxima
    x[7] = -4.0
    rows.append(x)
    x = (rng.standard_normal(k) * 1e-39).astype(np.float32)            # subnormal chunks
    x[::64] = 1e-37
    rows.append(x)
    x = (rng.standard_normal(k) * 1e36).astype(np.float32)             # near the top of f32
    rows.append(x)
    return rows


@pytest.mark.parametrize("n,k", [(300, 128), (896, 896), (4864, 896)])
def test_gemv_batch1_limb_activations_edge_values(plane, n, k):
    """The batch-1 group-32 GEMV against the float64 product of the dequantized weights on
    activations at the edges of the limb encoding, within the bound of the other GEMV tests
    (2e-6 * |W| |x|) plus the encoding's own: every element rounded to 2^-30 of its chunk's
    largest magnitude (2^-30 * |W| * chunkmax|x|). A NaN activation makes every output NaN, as
    in the f32 product."""
    q, s, deq = _quant(BH_Q4_G32, _w(n + 3 * k, n, k))
    dw = ops.DeviceWeight(plane, BH_Q4_G32, n, k, q, s)
    a64 = np.abs(deq).astype(np.float64)
    for i, x in enumerate(_limb_edge_rows(k)):
        y = dw.gemv(ops.DeviceArray.from_numpy(plane, x[None, :])).numpy()
        assert np.isfinite(y).all(), i
        want = x.astype(np.float64) @ deq.astype(np.float64).T
        cmax = np.repeat(np.abs(x.astype(np.float64)).reshape(-1, 32).max(axis=1), 32)
        bound = 2e-6 * (np.abs(x).astype(np.float64) @ a64.T) + 2.0 ** -30 * (cmax @ a64.T) + 1e-7
        assert np.all(np.abs(y[0] - want) <= bound), (i, float((np.abs(y[0] - want) / bound).max()))
    x = np.random.default_rng(1).standard_normal(k).astype(np.float32)
    x[k // 2] = np.nan
    y = dw.gemv(ops.DeviceArray.from_numpy(plane, x[None, :])).numpy()
    assert np.isnan(y).all()


@pytest.mark.parametrize("n,k", [(18944, 3584), (3584, 18944), (37000, 1024), (9999, 4096)])
def test_gemv_batch1_large_limb(plane, n, k):
    """Batch-1 group-32 GEMVs of 16 MiB and more on limb activations (K split over workgroups,
    partial sums of a tile added in split order) against the float64 product, at Qwen2-7B
    projection shapes and shapes whose K does not divide evenly into the splits; a second launch
    gives bit-identical results."""
    q, s, deq = _quant(BH_Q4_G32, _w(n + k, n, k))
    dw = ops.DeviceWeight(plane, BH_Q4_G32, n, k, q, s)
    x = np.random.default_rng(n).standard_normal((1, k)).astype(np.float32)
    xd = ops.DeviceArray.from_numpy(plane, x)
    y = dw.gemv(xd).numpy()
    _check_gemv(y, deq, x)
    assert np.array_equal(dw.gemv(xd).numpy().view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("fmt", [BH_Q4_G32, BH_Q4_ROW])
@pytest.mark.parametrize("n,k", [(37, 96), (300, 96), (1000, 896)])
@pytest.mark.parametrize("batch", [1, 9, 16, 32, 40, 63])
def test_gemv_ragged_rows(plane, fmt, n, k, batch):
    """Row counts that end inside a 64-row group (the padded rows and the group-32 scales of a
    partial group) through the VALU GEMV (batch 1), the MFMA passes (9..32 tokens) and the
    16-token-group passes (33..63)."""
    w = _w(fmt * 13 + n + k, n, k)
    q, s, deq = _quant(fmt, w)
    x = np.random.default_rng(n + batch).standard_normal((batch, k)).astype(np.float32)
    y = ops.DeviceWeight(plane, fmt, n, k, q, s).gemv(ops.DeviceArray.from_numpy(plane, x)).numpy()
    _check_gemv(y, deq, x)


@pytest.mark.parametrize("fmt", [BH_Q4_G32, BH_Q4_ROW])
@pytest.mark.parametrize("n,k,batch", [(896, 896, 64), (896, 896, 257), (4864, 896, 130), (896, 4864, 200), (300, 96, 71),
                                       (896, 896, 600), (18944, 896, 257), (896, 4864, 1031)])
def test_gemv_prefill_tiles(plane, fmt, n, k, batch):
    """Token counts of prefill chunks (>= 64): one tiled MFMA launch over all tokens with ragged
    row and token tiles where its grid fills the chip (18944 rows; 600 and 1031 tokens), else one
    launch of up to 32 16-token MFMA groups, with a K split over workgroups for long K."""
    w = _w(fmt * 17 + n + batch, n, k)
    q, s, deq = _quant(fmt, w)
    x = np.random.default_rng(batch).standard_normal((batch, k)).astype(np.float32)
    y = ops.DeviceWeight(plane, fmt, n, k, q, s).gemv(ops.DeviceArray.from_numpy(plane, x)).numpy()
    _check_gemv(y, deq, x)


@pytest.mark.parametrize("fmt", [BH_F32, BH_Q8_ROW, BH_Q4_ROW])
@pytest.mark.parametrize("n,k,batch", [(896, 896, 1), (4864, 896, 3), (896, 4864, 8), (300, 96, 5), (896, 4864, 20)])
def test_gemv_row_formats(plane, fmt, n, k, batch):
    w = _w(fmt * 31 + n, n, k)
    q, s, deq = _quant(fmt, w)
    x = np.random.default_rng(n).standard_normal((batch, k)).astype(np.float32)
    y = ops.DeviceWeight(plane, fmt, n, k, q, s).gemv(ops.DeviceArray.from_numpy(plane, x)).numpy()
    _check_gemv(y, deq, x)
    yo = oracle.matvec_mul_into(fmt, x[0], q, s, n)
    assert np.max(np.abs(y[0] - yo)) <= 1e-5 * max(1.0, np.abs(yo).max())


def test_matvec_mirror_reference_vectors(plane):
    # test_wgpu_gemv_vs_cpu (wgpu_backend.rs:1734-1782): GPU == CPU within 1e-4
    h = (np.arange(128, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    w = (np.arange(128 * 64, dtype=np.float32) * np.float32(0.0001)).astype(np.float32)
    gpu = plane.matvec_mul(h, w, 64)
    cpu = oracle.matvec_mul(oracle.F32, h, w.reshape(64, 128), None, 64)
    assert np.max(np.abs(gpu - cpu)) < 1e-4
    # test_quantization_correctness GPU branch (cpu_engine.rs:3649-3681)
    i = np.arange(64 * 128, dtype=np.float32)
    wq = (np.cos(i * np.float32(0.17)) * np.float32(0.5)).astype(np.float32).reshape(64, 128)
    hq = np.sin(np.arange(128, dtype=np.float32) * np.float32(0.31)).astype(np.float32)
    q8, s8 = oracle.quantize_int8(wq)
    assert np.max(np.abs(plane.matvec_mul_int8(hq, q8, s8, 64) - oracle.matvec_mul(oracle.Q8_ROW, hq, q8, s8, 64))) < 1e-4
    q4, s4 = oracle.quantize_int4(wq)
    assert np.max(np.abs(plane.matvec_mul_int4(hq, q4, s4, 64) - oracle.matvec_mul(oracle.Q4_ROW, hq, q4, s4, 64))) < 1e-4


def test_registry_errors_and_faults(plane):
    plane.clear_persistent_buffers()
    rng = np.random.default_rng(0)
    h = rng.standard_normal(896).astype(np.float32)
    w = _w(1, 896, 896)
    q, s = oracle.quantize_int4(w)
    want = oracle.matvec_mul_into(oracle.Q4_ROW, h, q, s, 896)
    y1 = plane.matvec_mul_int4(h, q, s, 896, "m", "layer.0")
    assert plane.registry_stats()[0] == 1
    # same key: the cached weight is used, the new argument's contents are ignored (get_or_create_op)
    y2 = plane.matvec_mul_int4(h, np.zeros_like(q), s, 896, "m", "layer.0")
    assert np.array_equal(y1, y2) and np.max(np.abs(y1 - want)) < 1e-4
    # same key, other shape: an error, not a wrong answer
    with pytest.raises(BhError):
        plane.matvec_mul_int4(h[:128], q[:, :64], s, 896, "m", "layer.0")
    # unkeyed calls do not register
    plane.matvec_mul_int4(h, q, s, 896)
    assert plane.registry_stats()[0] == 1
    # LRU eviction under the cap
    _, one = plane.registry_stats()
    plane.set_vram_cap(2 * one)
    plane.matvec_mul_int4(h, q, s, 896, "m", "layer.1")
    plane.matvec_mul_int4(h, q, s, 896, "m", "layer.0")  # touch 0: layer.1 is now oldest
    plane.matvec_mul_int4(h, q, s, 896, "m", "layer.2")
    n, b = plane.registry_stats()
    assert n == 2 and b <= 2 * one
    plane.set_vram_cap(64 << 30)
    plane.clear_persistent_buffers()
    assert plane.registry_stats() == (0, 0)
    # size mismatch -> Err(String) (wgpu_backend.rs:1096-1104)
    with pytest.raises(BhError, match="size mismatch"):
        plane.matvec_mul_int4(h, q[:-1], s, 896)
    # empty input -> Ok(zeros)
    assert np.array_equal(plane.matvec_mul(np.zeros(0, np.float32), np.zeros(0, np.float32), 5), np.zeros(5))
    # injected fault: the call fails without side effects, the next one succeeds, and the
    # dispatch seam hands the work back to the caller's CPU path
    plane.inject_fault(_lib.BH_OP_MATVEC, _lib.BH_ERR_INJECTED, 1)
    assert try_gpu_matvec(h, "int4", q, s, 896, plane=plane) is None
    assert np.max(np.abs(try_gpu_matvec(h, "int4", q, s, 896, plane=plane) - want)) < 1e-4


def test_rmsnorm_rope_silu(plane):
    D = lambda a: ops.DeviceArray.from_numpy(plane, a)  # noqa: E731
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((5, 896)) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(896)).astype(np.float32)
    got = ops.rmsnorm(plane, D(x), D(w), 1e-6).numpy()
    want = np.stack([oracle.rms_norm(r, w, 1e-6) for r in x])
    assert np.max(np.abs(got - want)) < 1e-5 * np.abs(want).max()
    pos = np.array([0, 1, 31, 4095, 32767], np.int32)
    v = rng.standard_normal((5, 14 * 64)).astype(np.float32)
    vt = D(v)
    ops.rope_(plane, vt, D(pos), 14, 64, 1e6, 40960)
    got = vt.numpy()
    for i, p in enumerate(pos):
        want = oracle.apply_rope(v[i], int(p), 14, 64, 1e6)
        assert np.max(np.abs(got[i] - want)) < 2e-6 * max(1.0, np.abs(want).max()), p
    g = (rng.standard_normal(4864) * 3).astype(np.float32)
    u = rng.standard_normal(4864).astype(np.float32)
    got = ops.silu_mul(plane, D(g), D(u)).numpy()
    want = oracle.silu_mul(g, u)
    assert np.max(np.abs(got - want)) < 2e-6 * np.abs(want).max()


def _attn_case(plane, lens, nq=14, nkv=2, hd=64, kv_f16=True, seed=0, check_rows=None, align=1):
    """Sequences at prefix-sum offsets (each capacity rounded up to `align` rows); every cache row
    outside the sequences is NaN, so a kernel that lets a stale row into a sum fails."""
    D = lambda a: ops.DeviceArray.from_numpy(plane, a)  # noqa: E731
    rng = np.random.default_rng(seed)
    B = len(lens)
    caps = [(n + align - 1) // align * align for n in lens]
    offs = np.concatenate([[0], np.cumsum(caps)[:-1]]).astype(np.int64)  # prefix sums
    rows = int(np.sum(caps))
    if kv_f16:
        rows = (rows + 63) // 64 * 64  # whole tiles
    k = np.full((nkv, rows, hd), np.nan, np.float32)
    v = np.full((nkv, rows, hd), np.nan, np.float32)
    for b in range(B):
        k[:, offs[b]:offs[b] + lens[b]] = rng.standard_normal((nkv, lens[b], hd))
        v[:, offs[b]:offs[b] + lens[b]] = rng.standard_normal((nkv, lens[b], hd))
    if kv_f16:
        k, v = k.astype(np.float16), v.astype(np.float16)
        kdev, vdev = ops.pack_kv_f16(k, v)
    else:
        kdev, vdev = k, v
    q = rng.standard_normal((B, nq * hd)).astype(np.float32)
    out = ops.attn_decode(plane, D(q), D(kdev), D(vdev), D(offs), D(np.array(lens, np.int32)), nq, nkv, hd,
                          int(max(lens))).numpy()
    assert np.all(np.isfinite(out))
    for b in (check_rows if check_rows is not None else range(B)):
        kc = k[:, offs[b]:offs[b] + lens[b]].astype(np.float32).transpose(1, 0, 2)  # -> [T][nkv][hd]
        vc = v[:, offs[b]:offs[b] + lens[b]].astype(np.float32).transpose(1, 0, 2)
        want = oracle.attn_decode(q[b], kc, vc, lens[b], nq, nkv, hd)
        assert np.max(np.abs(out[b] - want)) < 2e-5, (b, lens[b])


@pytest.mark.parametrize("T", [512, 4096, 32768])
@pytest.mark.parametrize("B", [1, 8])
def test_attention_config3(plane, T, B):
    # GQA 14 q / 2 kv heads, head_dim 64, fp16 K/V N(0,1), one query token, contexts 512/4096/32768
    _attn_case(plane, [T] * B, seed=T + B, check_rows=[0, B - 1])


def test_attention_ragged_and_short(plane):
    _attn_case(plane, [1, 2, 63, 64, 65, 200, 257, 1000], seed=1)  # unaligned offsets
    _attn_case(plane, [1, 2, 63, 64, 65, 200, 257, 1000], seed=4, align=8)  # 8-row aligned
    _attn_case(plane, [1, 2, 63, 64, 65, 200, 257, 1000], seed=5, align=64)  # whole tiles (decoder layout)
    _attn_case(plane, [130, 7, 64], nq=28, nkv=4, hd=128, seed=6, align=64)
    _attn_case(plane, [5, 300], kv_f16=False, seed=2)
    _attn_case(plane, [130, 7], nq=28, nkv=4, hd=128, seed=3)  # Qwen2-7B heads


def _attn_inputs(plane, B, T, seed, nq=14, nkv=2, hd=64):
    """Device inputs of a batch of B sequences of T rows (fp16 tile layout, 64-row regions)."""
    D = lambda a: ops.DeviceArray.from_numpy(plane, a)  # noqa: E731
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((nkv, B * T, hd)).astype(np.float16)
    v = rng.standard_normal((nkv, B * T, hd)).astype(np.float16)
    kp, vp = ops.pack_kv_f16(k, v)
    q = rng.standard_normal((B, nq * hd)).astype(np.float32)
    offs = (np.arange(B) * T).astype(np.int64)
    return [D(q), D(kp), D(vp), D(offs), D(np.full(B, T, np.int32))]


def test_attention_on_two_streams_keeps_split_scratch_apart(plane):
    """Split attention calls queued on two caller streams at once (no synchronisation between
    them) each use their own stream's partials and merge counters: every output equals the same
    call made alone on the context's stream."""
    import ctypes

    from bramha_amd._lib import check, lib

    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime the library already loaded (same soname)
    streams = [ctypes.c_void_p(), ctypes.c_void_p()]
    for s in streams:
        assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    nq, nkv, hd, T, B = 14, 2, 64, 4096, 8
    ins = [_attn_inputs(plane, B, T, seed=70 + i) for i in range(2)]
    want = [ops.attn_decode(plane, *x, nq, nkv, hd, T).numpy() for x in ins]
    outs = [[ops.DeviceArray(plane, (B, nq * hd), np.float32) for _ in range(6)] for _ in range(2)]
    for r in range(6):
        for i in range(2):
            q, k, v, off, ln = ins[i]
            check(lib.bh_attn_decode(plane.ctx, q.ptr, k.ptr, v.ptr, 1, B * T, off.ptr, ln.ptr, B, nq, nkv, hd, T,
                                     outs[i][r].ptr, streams[i]), plane.ctx)
    ops.synchronize(plane)
    for i in range(2):
        for r in range(6):
            assert np.array_equal(outs[i][r].numpy(), want[i]), (i, r)
    for s in streams:
        assert hip.hipStreamDestroy(s) == 0


def test_probes_run_and_reject_bad_shapes(plane):
    """The measurement probes behind the bench's floor figures: a dependent-launch chain link and a
    grid-barrier phase over a resident grid (every wait bounded; a wait that gave up would fail the
    call) both time, and a grid-barrier probe wider than one workgroup per CU is refused."""
    assert ops.time_probe(plane, 2, 896 * 4, 14, 4, iters=8) > 0
    for wgs in (1, 14, 256):
        assert ops.time_probe(plane, 3, 4096, wgs, 4, iters=4) > 0
    with pytest.raises(BhError):
        ops.time_probe(plane, 3, 4096, 1 << 16, 4, iters=1)
