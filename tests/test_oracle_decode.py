"""Pins of the decode-step oracle (oracle/heph_decode_oracle.c), CPU only.

Each op is checked against closed forms and an independent float64 numpy
restatement of the reference's formula (forward.mojo:45-81, kernels.mojo:
530-548, :709-762, :923-1035, :1243-1255, :1376-1433), with cases chosen
so that a dropped term, a wrong index or a swapped operand fails.
"""
import numpy as np
import pytest

from oracle import oracle as O

ULP = 2.0 ** -8      # bf16 relative step (8 significant bits)


def bf16(x):
    return O.f32_to_bf16(np.ascontiguousarray(x, np.float32))


def f32(b):
    return O.bf16_to_f32(np.ascontiguousarray(b, np.uint16)).astype(np.float64)


def rng_bf16(seed, n, scale=1.0):
    return bf16(np.random.default_rng(seed).standard_normal(n) * scale)


# ------------------------------------------------------------------ embed ----

def test_embed_block_and_channel_scales():
    V, H = 300, 256
    rng = np.random.default_rng(0)
    emb = rng.integers(0, 0x7E, size=(V, H), dtype=np.uint8)
    emb[:, ::7] |= 0x80                                   # negative codes too
    # power-of-two block scales: a wrong block index changes the exponent
    sblk = (2.0 ** rng.integers(-6, 6, size=(-(-V // 128), H // 128))).astype(np.float32)
    schan = (2.0 ** rng.integers(-6, 6, size=V)).astype(np.float32)
    dec = O.e4m3_decode_table().astype(np.float64)
    toks = [0, 127, 128, 299]
    x = O.embed_fp8(emb, sblk, True, toks)
    for i, t in enumerate(toks):
        want = bf16(dec[emb[t]] * np.repeat(sblk[t // 128], 128))
        assert np.array_equal(x[i], want)
    x = O.embed_fp8(emb, schan, False, toks)
    for i, t in enumerate(toks):
        assert np.array_equal(x[i], bf16(dec[emb[t]] * schan[t]))


# ---------------------------------------------------------------- rmsnorm ----

def hf_rmsnorm64(x, gamma, eps=1e-6):
    x = f32(x)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return f32(gamma) * f32(bf16(y))


def test_rmsnorm_constant_row_and_gamma():
    g = rng_bf16(1, 2560)
    for c in (3.0, -0.5, 1e-3):
        x = bf16(np.full(2560, c))
        y = f32(O.rmsnorm(x, g))
        # x / rms(x) = sign(c) (eps negligible except for the tiny row)
        want = f32(g) * f32(bf16(np.full(2560, np.sign(c) / np.sqrt(1 + 1e-6 / (c * c)))))
        assert np.allclose(y, want, rtol=2 * ULP, atol=0)


@pytest.mark.parametrize("cols,scale", [(2560, 1.0), (2560, 1e-3), (9728, 30.0), (128, 1.0)])
def test_rmsnorm_vs_float64(cols, scale):
    x = rng_bf16(cols, 3 * cols, scale).reshape(3, cols)
    g = rng_bf16(cols + 1, cols)
    y = f32(O.rmsnorm(x, g))
    ref = hf_rmsnorm64(x, g)
    assert np.all(np.abs(y - ref) <= 2 * ULP * np.abs(ref) + 1e-30)
    # mean (not sum) of squares, and gamma applied after the bf16 cast
    assert not np.allclose(y, f32(g) * f32(x) / np.sqrt(np.sum(f32(x) ** 2, -1, keepdims=True)))


# ------------------------------------------------------------------- rope ----

def rope_cs64(pos, p, D=128, theta=1e6):
    freq = np.float32(pos * theta ** (-2.0 * p / D))
    c = float(f32(bf16(np.float32(np.cos(np.float64(freq))))).reshape(-1)[0])
    s = float(f32(bf16(np.float32(np.sin(np.float64(freq))))).reshape(-1)[0])
    return c, s


def test_rope_table():
    for pos in (0, 1, 4096, 123457):
        for p in (0, 1, 17, 63):
            assert O.rope_cs(pos, p) == rope_cs64(pos, p), (pos, p)
    assert all(O.rope_cs(0, p) == (1.0, 0.0) for p in range(64))
    # theta enters as theta^(-2p/D): p = 0 is independent of theta
    assert O.rope_cs(777, 0, theta=5e6) == O.rope_cs(777, 0, theta=1e6)
    assert O.rope_cs(777, 9, theta=5e6) != O.rope_cs(777, 9, theta=1e6)


def qk64(qkv, qg, kg, inv, NH, NKV, pos):
    """float64 restatement: per-head norm, then split-half rotation with
    bf16 rounding after every op, then E4M3 for k and v."""
    D = 128
    heads = f32(qkv).reshape(-1, D)
    q_out, k_codes, v_codes = [], [], []
    for h in range(NH + 2 * NKV):
        row = heads[h]
        if h >= NH + NKV:
            v = np.clip(row * inv[NKV + h - NH - NKV], -448, 448)
            v_codes.append(O.e4m3_encode(v.astype(np.float32)))
            continue
        g = f32(qg if h < NH else kg)
        y = f32(bf16(g * f32(bf16(row / np.sqrt(np.mean(row * row) + 1e-6)))))
        a, b = y[:64], y[64:]
        cs = np.array([rope_cs64(pos, p) for p in range(64)])
        c, s = cs[:, 0], cs[:, 1]
        rb = lambda t: f32(bf16(t))
        re = rb(rb(a * c) - rb(b * s))
        im = rb(rb(b * c) + rb(a * s))
        out = np.concatenate([re, im])
        if h < NH:
            q_out.append(out)
        else:
            k = np.clip(out * inv[h - NH], -448, 448)
            k_codes.append(O.e4m3_encode(k.astype(np.float32)))
    return np.concatenate(q_out), np.concatenate(k_codes), np.concatenate(v_codes)


@pytest.mark.parametrize("pos", [0, 5, 4096])
def test_qk_norm_rope_kv_vs_float64(pos):
    NH, NKV = 4, 2
    qkv = rng_bf16(pos + 3, (NH + 2 * NKV) * 128, 2.0)
    qg, kg = rng_bf16(11, 128), rng_bf16(12, 128)
    inv = np.array([40.0, 30.0, 20.0, 500.0], np.float32)   # last one saturates some v
    q, k, v = O.qk_norm_rope_kv(qkv, qg, kg, inv, NH, NKV, pos)
    q64, k64, v64 = qk64(qkv, qg, kg, inv, NH, NKV, pos)
    # the squared-norm sum order differs from float64: allow one bf16 step
    assert np.all(np.abs(f32(q) - q64) <= 2 * ULP * np.abs(q64) + 1e-6)
    assert np.mean(f32(q) == q64) > 0.98
    assert np.array_equal(v, v64)
    assert np.mean(k == k64) > 0.98
    assert np.any(v[128:] == 0x7E) and np.any(v[128:] == 0xFE)     # saturated, not NaN
    if pos == 0:      # identity rotation: q is just the normalized head
        qn = np.concatenate([f32(bf16(f32(qg) * f32(bf16(r / np.sqrt(np.mean(r * r) + 1e-6)))))
                             for r in f32(qkv).reshape(-1, 128)[:NH]])
        assert np.allclose(f32(q), qn, rtol=2 * ULP, atol=1e-6)


# -------------------------------------------------------------- attention ----

def attention64(q, kc, vc, scale, NH, NKV, n):
    dec = O.e4m3_decode_table().astype(np.float64)
    out = []
    for h in range(NH):
        kh = h // (NH // NKV)
        qq = f32(q[h * 128:(h + 1) * 128])
        K = dec[kc[:n, kh]] * scale[kh]
        V = dec[vc[:n, kh]] * scale[NKV + kh]
        s = K @ qq / np.sqrt(128.0)
        p = np.exp(s - s.max())
        p = f32(bf16(p / p.sum()))
        out.append(p @ V)
    return np.concatenate(out)


@pytest.mark.parametrize("n", [1, 2, 300, 4097])
def test_attention_vs_float64(n):
    NH, NKV = 4, 2
    rng = np.random.default_rng(n)
    q = rng_bf16(n, NH * 128, 3.0)
    kc = rng.integers(0, 0x7E, size=(n, NKV, 128), dtype=np.uint8) | \
        (rng.integers(0, 2, size=(n, NKV, 128), dtype=np.uint8) << 7)
    vc = rng.integers(0, 0x7E, size=(n, NKV, 128), dtype=np.uint8) | \
        (rng.integers(0, 2, size=(n, NKV, 128), dtype=np.uint8) << 7)
    scale = np.array([0.01, 0.02, 0.03, 0.04], np.float32)
    got = f32(O.attention_fp8kv(q, kc, vc, scale, NH, NKV, n))
    ref = attention64(q, kc, vc, scale, NH, NKV, n)
    tol = 4 * ULP * np.abs(ref).max()
    assert np.all(np.abs(got - ref) <= tol), np.abs(got - ref).max() / tol
    if n == 1:          # a single key: p = 1 and out = bf16(v * sv) exactly
        dec = O.e4m3_decode_table()
        want = np.concatenate([bf16(dec[vc[0, h // 2]] * scale[2 + h // 2]) for h in range(NH)])
        # (values compared, so the accumulator's +0 equals a -0 code)
        assert np.array_equal(f32(O.attention_fp8kv(q, kc, vc, scale, NH, NKV, 1)), f32(want))


def test_attention_gqa_head_mapping():
    # query heads 0,1 read kv head 0 and heads 2,3 kv head 1 (h // group)
    NH, NKV, n = 4, 2, 3
    q = rng_bf16(5, NH * 128)
    kc = np.zeros((n, NKV, 128), np.uint8)
    vc = np.zeros((n, NKV, 128), np.uint8)
    vc[:, 0] = 0x38      # 1.0
    vc[:, 1] = 0x40      # 2.0
    out = f32(O.attention_fp8kv(q, kc, vc, np.ones(4, np.float32), NH, NKV, n)).reshape(NH, 128)
    p = f32(bf16(np.float32(1.0 / 3.0)))          # uniform scores
    assert np.allclose(out[:2], 3 * p * 1.0, rtol=ULP) and np.allclose(out[2:], 3 * p * 2.0,
                                                                         rtol=ULP)


# ----------------------------------------------------------- silu, argmax ----

def test_silu_mul_vs_float64():
    g = rng_bf16(21, 9728, 4.0)
    u = rng_bf16(22, 9728)
    got = f32(O.silu_mul(g, u))
    gg = f32(g)
    silu = f32(bf16(gg / (1 + np.exp(-gg))))
    ref = silu * f32(u)
    assert np.all(np.abs(got - ref) <= 2 * ULP * np.abs(ref) + 1e-30)
    assert np.all(O.silu_mul(bf16(np.zeros(4)), bf16(np.ones(4))) == 0)
    # silu is applied to gate, not up
    assert not np.allclose(got, f32(bf16(f32(u) / (1 + np.exp(-f32(u))))) * gg)


def test_argmax_lowest_index_on_bf16_ties():
    x = np.zeros(1000, np.float32)
    x[[17, 500, 999]] = 5.0
    assert O.argmax_bf16(x) == 17
    x = np.zeros(1000, np.float32)
    x[900] = 1.0
    x[100] = 1.0 + 2.0 ** -12          # larger in f32, same value in bf16
    assert O.argmax_bf16(x) == 100
    x[50] = 1.0 + 2.0 ** -13
    assert O.argmax_bf16(x) == 50
    x[60] = 1.0 + 2.0 ** -7            # a real bf16 step above
    assert O.argmax_bf16(x) == 60
