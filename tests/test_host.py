"""CPU tests of the product library's host side: it loads and exports every symbol the
header declares, its synthetic generator matches an independent numpy restatement, its
quantizers are bit-identical to the oracle's (the reference's), and the dispatch policy
keeps the caller on its CPU path when no device is usable."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
import ref64
from bramha_amd import _lib
from bramha_amd.model import quantize, synth_normal, synth_tokens
from bramha_amd.plane import CPU, GPU, route_op, try_gpu_matvec

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "bramha_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(_lib.lib, n)]
    assert not missing, missing
    assert set(names) <= set(_lib._PROTOS), "binding lacks prototypes for declared symbols"


def test_init_without_device_is_an_error_not_a_crash():
    h = ctypes.c_void_p()
    assert _lib.lib.bh_init(0, None) == _lib.BH_ERR_INVALID
    assert _lib.lib.bh_init(-1, ctypes.byref(h)) == _lib.BH_ERR_NO_DEVICE
    import torch

    if torch.cuda.device_count() == 0:
        assert _lib.lib.bh_init(0, ctypes.byref(h)) == _lib.BH_ERR_NO_DEVICE
        assert h.value is None
    assert _lib.lib.bh_status_str(_lib.BH_ERR_CAPACITY) == b"capacity exceeded"
    assert _lib.lib.bh_last_error(None) == b"no context"


def test_synth_normal_matches_numpy_restatement():
    for name, n in (("model.layers.0.mlp.up_proj.weight", 100001), ("x", 7)):
        got = synth_normal(1234, name, n, 0.02)
        want = ref64.synth_normal_np(1234, name, n, 0.02)
        diff = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
        assert diff.max() <= 1 and (diff == 0).mean() > 0.9999  # libm cos/log may differ by 1 ulp
        assert abs(float(got.std()) - 0.02) < 0.001 if n > 1000 else True
    a = synth_normal(1, "a", 1000, 1.0)
    assert not np.array_equal(a, synth_normal(2, "a", 1000, 1.0))
    assert not np.array_equal(a, synth_normal(1, "b", 1000, 1.0))
    t = synth_tokens(7, "prompt", 10000, 151936)
    assert t.dtype == np.uint32 and t.max() < 151936 and len(np.unique(t)) > 9000


@pytest.mark.parametrize("n,k", [(64, 128), (33, 896), (4, 4864)])
def test_product_quantizers_bit_identical_to_oracle(n, k):
    rng = np.random.default_rng(n)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[1] = 0
    w[2, :16] = np.float32(2.5)  # exact .5 quotients
    q, s = quantize(_lib.BH_Q8_ROW, w)
    oq, os_ = oracle.quantize_int8(w)
    assert np.array_equal(q, oq) and np.array_equal(s.view(np.uint32), os_.view(np.uint32))
    q, s = quantize(_lib.BH_Q4_ROW, w)
    oq, os_ = oracle.quantize_int4(w)
    assert np.array_equal(q, oq) and np.array_equal(s.view(np.uint32), os_.view(np.uint32))
    q, s = quantize(_lib.BH_Q4_G32, w)
    oq, os_ = oracle.quantize_q4g32(w)
    assert np.array_equal(q, oq) and np.array_equal(s, os_)


def test_route_op_mirrors_scheduler():
    # HeterogeneousScheduler::route_op (scheduler.rs:31-62)
    assert route_op(10**6, "gemv", gpu_available=True, force_cpu=False) == GPU
    assert route_op(131071, "gemv", gpu_available=True, force_cpu=False) == CPU
    assert route_op(262144, "gemm", gpu_available=True, force_cpu=False) == GPU
    assert route_op(262143, "gemm", gpu_available=True, force_cpu=False) == CPU
    assert route_op(10**9, "embedding", gpu_available=True, force_cpu=False) == CPU
    assert route_op(10**9, "sampling", gpu_available=True, force_cpu=False) == CPU
    assert route_op(10**9, "attention", gpu_available=True, force_cpu=False) == GPU
    assert route_op(10**9, "gemv", gpu_available=True, force_cpu=True) == CPU
    assert route_op(10**9, "gemv", gpu_available=False, force_cpu=False) == CPU


def test_cpu_only_mode_falls_back(monkeypatch):
    from bramha_amd import plane as pl

    monkeypatch.setenv("BRAMHA_CPU", "1")
    assert pl.get_hip_plane() is None
    h = np.ones(896, np.float32)
    w = np.ones((896, 896), np.float32)
    assert try_gpu_matvec(h, "f32", w, None, 896) is None  # the caller runs its CPU GEMV


def test_kv_tile_layout():
    """The fp16 cache layout is a permutation of each head's region, and the first operand of a
    tile — MFMA block 0 / chunk 0 for K, row group 0 / dim block 0 for V — is lane-ordered: lane
    (lr, lg) = lane % 16, lane // 16 holds its 8 elements at offsets 8 lane .. 8 lane + 7."""
    import numpy as np

    from bramha_amd import ops

    for hd in (64, 128):
        ki, vi = ops.kv_tile_index(128, hd)
        for idx in (ki, vi):
            assert np.array_equal(np.sort(idx.ravel()), np.arange(128 * hd))
        for lane in range(64):
            lr, lg = lane % 16, lane // 16
            row = 8 * (lr >> 2) + (lr & 3)  # row of block 0, lane-group row lr
            assert list(ki[row, 8 * lg:8 * lg + 8]) == list(range(8 * lane, 8 * lane + 8))
            assert list(vi[8 * lg:8 * lg + 8, lr]) == list(range(8 * lane, 8 * lane + 8))
