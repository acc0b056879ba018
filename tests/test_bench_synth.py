"""bench.py's synthetic inputs (libhephbench.so, bench_csrc/synth.cpp) are the
sequence of the parity tests' seeded generator: bit for bit the oracle's
normal and activation streams for the same seeds and offsets, and the same
FNV-1a digest. The bench's committed input digests follow from them."""
import ctypes
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

LIB = os.path.join(os.path.dirname(__file__), "..", "hephaestus_amd", "libhephbench.so")


@pytest.fixture(scope="module")
def blib():
    if not os.path.exists(LIB):
        pytest.skip("libhephbench.so not built")
    lib = ctypes.CDLL(LIB)
    u64, sz, f32, f64 = ctypes.c_uint64, ctypes.c_size_t, ctypes.c_float, ctypes.c_double
    vp = ctypes.c_void_p
    lib.heph_bench_gen_normal.argtypes = [u64, u64, sz, f32, f32, vp]
    lib.heph_bench_gen_normal_bf16.argtypes = [u64, u64, sz, f32, f32, vp]
    lib.heph_bench_gen_act_bf16.argtypes = [u64, sz, f64, f32, vp]
    lib.heph_bench_fnv1a64.argtypes = [vp, sz]
    lib.heph_bench_fnv1a64.restype = u64
    return lib


@pytest.mark.parametrize("seed,offset,n,mean,std", [(0, 0, 1 << 17, 0.0, 0.02),
                                                   (7, 12345, 70001, 0.0, 1.0),
                                                   (2 ** 63 + 11, 3, 999, 1.0, 0.1)])
def test_normal_stream_equals_oracle(blib, seed, offset, n, mean, std):
    got = np.empty(n, np.float32)
    blib.heph_bench_gen_normal(seed, offset, n, mean, std, got.ctypes.data)
    want = O.gen_normal(seed, n, mean, std, offset=offset)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    bf = np.empty(n, np.uint16)
    blib.heph_bench_gen_normal_bf16(seed, offset, n, mean, std, bf.ctypes.data)
    assert np.array_equal(bf, O.f32_to_bf16(want))


@pytest.mark.parametrize("seed,M,K,p", [(0, 1, 2560, 0.0), (4097, 64, 9728, 1e-3),
                                        (513, 300, 4096, 1e-3)])
def test_activation_stream_equals_oracle(blib, seed, M, K, p):
    got = np.empty(M * K, np.uint16)
    blib.heph_bench_gen_act_bf16(seed, M * K, p, 50.0, got.ctypes.data)
    want = O.gen_act_bf16(seed, M, K, outlier_p=p).reshape(-1)
    assert np.array_equal(got, want)
    if p:
        assert (np.abs(O.bf16_to_f32(got)) > 6.0).sum() > 0      # the outliers are there
    assert blib.heph_bench_fnv1a64(got.ctypes.data, got.nbytes) == int(O.digest(got), 16)


def test_bench_config0_activation_is_the_parity_row(golden_dir):
    # configs[0]'s activation row is the parity tests' seed-0 row
    import bench
    d = json.load(open(os.path.join(golden_dir, "digests.json")))
    assert bench.CONFIG0_SEED == 0
    assert bench.BENCH_DIGESTS["x_config0"] == d["x_config0"]
    assert O.digest(O.gen_act_bf16(bench.CONFIG0_SEED, 1, 2560)) == d["x_config0"]


def test_bench_input_digests(blib):
    # every digest bench.py checks on the GPU box follows from the generator
    # and the weight quantizer (the library's is bit-exact with the oracle's
    # on bf16 input); the lm_head's bf16 weights (778 MB) are digested as
    # generated, unquantized
    import bench
    want = bench.BENCH_DIGESTS
    seen = set()
    for name, N, K in bench.SHAPES + [bench.Q_PROJ]:
        w = np.empty(N * K, np.uint16)
        blib.heph_bench_gen_normal_bf16(bench.WEIGHT_SEEDS[name], 0, N * K, 0.0, 0.02,
                                        w.ctypes.data)
        assert O.digest(w) == want[f"{name}_w_bf16"], name
        qw, sw = O.quant_weight(O.bf16_to_f32(w).reshape(N, K), 128, 128)
        assert O.digest(qw) == want[f"{name}_w_e4m3"], name
        assert O.digest(sw) == want[f"{name}_scale_inv"], name
        seen |= {f"{name}_w_bf16", f"{name}_w_e4m3", f"{name}_scale_inv"}
    name, N, K = bench.LM_HEAD
    w = np.empty(N * K, np.uint16)
    blib.heph_bench_gen_normal_bf16(bench.WEIGHT_SEEDS[name], 0, N * K, 0.0, 0.02,
                                    w.ctypes.data)
    assert O.digest(w) == want["lm_head_w_bf16"]
    del w
    seen.add("lm_head_w_bf16")
    for K in {K for _, _, K in bench.SHAPES}:
        assert O.digest(O.gen_act_bf16(K, 1, K)) == want[f"x_m1_k{K}"], K
        seen.add(f"x_m1_k{K}")
    seen.add("x_config0")
    assert seen == set(want)
