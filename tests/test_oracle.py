"""The oracle pinned: golden outputs of qw6's own CPU path, the reference
build itself where present, and closed forms / known-answer constructions of
qw6's self-tests (restated, with their tolerances)."""
import hashlib
from pathlib import Path

import numpy as np
import pytest

import cases
import oracle as O
from qw6_amd import synth as S

G = np.load(Path(__file__).parent / "golden" / "golden.npz")
FORMATS = [S.Q_Q4_K_M, S.Q_Q5_K, S.Q_Q6_K, S.Q_IQ2_XXS, S.Q_IQ2_S, S.Q_IQ3_S]
MV_SHAPES = [(3, 256), (16, 512), (8, 2048), (5, 1280)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fp16_exhaustive_closed_form_and_golden():
    h = np.arange(65536, dtype=np.uint16)
    got = np.array([O.fp16_to_f32(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)      # IEEE binary16 -> binary32
    ok = ~np.isnan(want)
    assert np.array_equal(bits(got)[ok], bits(want)[ok])
    assert np.isnan(got[~ok]).all()
    assert hashlib.sha256(got.tobytes()).digest() == bytes(G["fp16_sha256"])


def test_scale_min_k4_brute_force():
    """All 6-bit (sc, m) pairs round-trip through the 12-byte packing."""
    import ctypes as C
    rng = np.random.default_rng(0)
    for _ in range(200):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        q = np.zeros(12, np.uint8)
        for j in range(4):
            q[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
            q[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
            q[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
        for j in range(8):
            d, mm = C.c_uint8(), C.c_uint8()
            O.lib().orc_scale_min_k4(j, q.ctypes.data, C.addressof(d), C.addressof(mm))
            assert (d.value, mm.value) == (sc[j], m[j])


TABLE_SHA = {  # SHA-256 of the reference tables' little-endian byte images
    "kmask": "5ac9831b2e30eb285ef34f8501620f878432d5c04331ad1ae47f977a83ba41a5",
    "ksigns": "a76742a603f8beca5212ecce0f1f02f11a4887fd2f7c8b15aca0ea3eb3380c31",
    "iq2xxs": "05826b5d3e472a3a78f196be62ac78acf81df0f909626e12ab9fa2a5d490dd54",
    "iq2s": "e1aa1473412b0552c2174c30ef22ab4073f6a181b85a17056e8249bd2932fd88",
    "iq3s": "bd1af4945a1717c65610b0284e4628b9a1ba3b306fae3a06f6e5f597356e349f",
}


def test_iq_tables_match_reference_images():
    i2 = np.zeros(256, np.uint64); i2s = np.zeros(1024, np.uint64)
    i3 = np.zeros(512, np.uint32); ks = np.zeros(128, np.uint8); km = np.zeros(8, np.uint8)
    O.lib().orc_iq_tables(i2.ctypes.data, i2s.ctypes.data, i3.ctypes.data, ks.ctypes.data,
                          km.ctypes.data)
    for name, arr in (("kmask", km), ("ksigns", ks), ("iq2xxs", i2), ("iq2s", i2s), ("iq3s", i3)):
        assert hashlib.sha256(arr.tobytes()).hexdigest() == TABLE_SHA[name], name
    # invariants: lattice bytes
    b2 = np.concatenate([i2.view(np.uint8), i2s.view(np.uint8)])
    assert set(np.unique(b2)) == {0x08, 0x19, 0x2B}
    assert set(np.unique(i3.view(np.uint8))) == set(range(1, 16, 2))
    # even parity of every sign byte
    assert all(bin(int(v)).count("1") % 2 == 0 for v in ks)


@pytest.mark.parametrize("q", FORMATS)
@pytest.mark.parametrize("shape", MV_SHAPES)
def test_matvec_bitwise_golden(q, shape):
    rows, cols = shape
    w = S.quant_matrix(3, S.stream_id(0, S.K_GATE, q), q, rows, cols)
    x = S.f32_normal(3, S.stream_id(0, S.K_X, q), cols, 1.0)
    y = O.matvec(q, w, rows, cols, x)
    assert np.array_equal(bits(y), bits(G["mv_%d_%dx%d" % (q, rows, cols)]))
    # the multi-threaded variant keeps per-row order: bit-identical
    assert np.array_equal(bits(O.matvec(q, w, rows, cols, x, nthreads=3)), bits(y))


@pytest.mark.parametrize("q", FORMATS)
def test_dequant_golden(q):
    w = S.quant_matrix(5, S.stream_id(0, S.K_UP, q), q, 2, 512)
    got = np.stack([O.dequant_row(q, w, 512, r) for r in range(2)])
    assert np.array_equal(bits(got), bits(G["deq_%d" % q]))


def test_cfg0_golden():
    w = S.quant_matrix(1, S.stream_id(0, S.K_GATE), S.Q_Q4_K_M, 512, 2048)
    x = S.f32_normal(1, S.stream_id(0, S.K_X), 2048, 1.0)
    assert np.array_equal(bits(O.matvec(S.Q_Q4_K_M, w, 512, 2048, x)), bits(G["cfg0_y"]))


def test_unsupported_quant_fails():
    w = np.zeros(144 * 2, np.uint8)
    with pytest.raises(ValueError):
        O.matvec(S.Q_IQ2_XXS + 5, w, 2, 256, np.zeros(256, np.float32))
    assert O.lib().orc_dequant_row(3, w.ctypes.data, 256, 0, np.zeros(256, np.float32)) == -1


# ---- known-answer constructions of qw6's Vulkan self-test, restated -------------

def put_u16(b, off, v):
    b[off] = v & 0xFF
    b[off + 1] = v >> 8


def test_kat_q4k():
    """qw6_vk.c:1609-1649: d=1, dmin=0, unit scales, patterned nibbles."""
    rows, cols = 3, 256
    x = np.sin(np.arange(cols, dtype=np.float32) * np.float32(0.031)).astype(np.float32)
    w = np.zeros((rows, 144), np.uint8)
    want = np.zeros(rows)
    for r in range(rows):
        put_u16(w[r], 0, 0x3C00)
        for j in range(8):
            if j < 4:
                w[r, 4 + j] = 1
            else:
                w[r, 8 + j] = 1
        for c in range(cols):
            g64, sub = c >> 6, (c >> 5) & 1
            off = 16 + g64 * 32 + (c & 31)
            qv = (r * 3 + c * 5 + 7) & 15
            w[r, off] = (w[r, off] & 0xF0) | qv if sub == 0 else (w[r, off] & 0x0F) | (qv << 4)
            want[r] += qv * x[c]   # every sub-block scale is 1
    y = O.matvec(S.Q_Q4_K_M, w.reshape(-1), rows, cols, x)
    assert np.abs(y - want).max() < 1e-2


def test_kat_q5k():
    """qw6_vk.c:1651-1704: 5-bit codes with the high bit in qh."""
    rows, cols = 3, 256
    x = np.cos(np.arange(cols, dtype=np.float32) * np.float32(0.027)).astype(np.float32)
    w = np.zeros((rows, 176), np.uint8)
    want = np.zeros(rows)
    for r in range(rows):
        put_u16(w[r], 0, 0x3C00)
        for j in range(8):
            if j < 4:
                w[r, 4 + j] = 1
            else:
                w[r, 8 + j] = 1
        for c in range(cols):
            g64, sub, lane = c >> 6, (c >> 5) & 1, c & 31
            off = 48 + g64 * 32 + lane
            qv = (r * 7 + c * 3 + 5) & 31
            w[r, off] = (w[r, off] & 0xF0) | (qv & 15) if sub == 0 else (w[r, off] & 0x0F) | ((qv & 15) << 4)
            if qv & 16:
                w[r, 16 + lane] |= 1 << (g64 * 2 + sub)
            want[r] += qv * x[c]
    y = O.matvec(S.Q_Q5_K, w.reshape(-1), rows, cols, x)
    assert np.abs(y - want).max() < 1e-2


def test_kat_q6k():
    """qw6_vk.c:1706-1742 (all scales 1), plus distinct scales to pin qw6's
    even-scale rule: the run k of half h uses scales[8h + 2k]."""
    rows, cols = 3, 256
    c_ = np.arange(cols, dtype=np.float32)
    x = (np.sin(c_ * np.float32(0.019)) + np.float32(0.2) * np.cos(c_ * np.float32(0.013))).astype(np.float32)
    w = np.zeros((rows, 210), np.uint8)
    qvs = np.zeros((rows, cols))
    for r in range(rows):
        put_u16(w[r], 208, 0x3C00)
        w[r, 192:208] = 1
        for c in range(cols):
            half, in_half = c >> 7, c & 127
            lane, quad = in_half & 31, in_half >> 5
            qv = ((r * 11 + c * 7 + 9) & 63) - 32
            u = qv + 32
            ql_off = half * 64 + lane + (32 if quad in (1, 3) else 0)
            qh_off = 128 + half * 32 + lane
            w[r, ql_off] = (w[r, ql_off] & 0xF0) | (u & 15) if quad < 2 else (w[r, ql_off] & 0x0F) | ((u & 15) << 4)
            w[r, qh_off] |= ((u >> 4) & 3) << (quad * 2)
            qvs[r, c] = qv
    y = O.matvec(S.Q_Q6_K, w.reshape(-1), rows, cols, x)
    assert np.abs(y - qvs @ x).max() < 1e-2
    # distinct scales: 1..16 -> even-only rule
    w[:, 192:208] = np.arange(1, 17, dtype=np.uint8)
    sc = np.zeros(cols)
    for c in range(cols):
        h, k = c >> 7, (c & 127) >> 5
        sc[c] = 8 * h + 2 * k + 1
    y = O.matvec(S.Q_Q6_K, w.reshape(-1), rows, cols, x)
    assert np.abs(y - (qvs * sc) @ x).max() < 1e-1


def test_kat_iq2xxs():
    """qw6_vk.c:1744-1787: grid index 0, no signs, no scale -> every weight d."""
    rows, cols = 3, 256
    c_ = np.arange(cols, dtype=np.float32)
    x = (np.sin(c_ * np.float32(0.029)) + np.float32(0.15) * np.cos(c_ * np.float32(0.017))).astype(np.float32)
    w = np.zeros((rows, 66), np.uint8)
    for r, hv in enumerate((0x3C00, 0x3E00, 0x4000)):
        put_u16(w[r], 0, hv)
    y = O.matvec(S.Q_IQ2_XXS, w.reshape(-1), rows, cols, x)
    want = np.array([1.0, 1.5, 2.0]) * x.astype(np.float64).sum()
    assert np.abs(y - want).max() < 2e-2


def test_kat_iq2s_iq3s_closed_form():
    """All-zero indices: IQ2_S weight = d*0.125*8 = d (scale nibble 0);
    IQ3_S weight = d*(1+0)*1 = d (grid entry 0 is 0x01010101)."""
    x = np.linspace(-1, 1, 256).astype(np.float32)
    for q, nb in ((S.Q_IQ2_S, 82), (S.Q_IQ3_S, 110)):
        w = np.zeros(nb, np.uint8)
        put_u16(w, 0, 0x4000)   # d = 2
        y = O.matvec(q, w, 1, 256, x)
        assert abs(y[0] - 2.0 * x.astype(np.float64).sum()) < 1e-4


def test_kat_matvec_f32():
    """qw6_vk.c:1585-1607: 7 x 19 dense F32."""
    rows, cols = 7, 19
    r_, c_ = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    w = (np.float32(0.01) * (r_ - c_)).astype(np.float32)
    x = np.cos(np.arange(cols, dtype=np.float32) * np.float32(0.2)).astype(np.float32)
    y = O.matvec(S.Q_FP32, w.reshape(-1), rows, cols, x)
    assert np.abs(y - w.astype(np.float64) @ x).max() < 2e-5


@pytest.mark.parametrize("name", ["route_randn", "route_ties", "route_small", "route_vkkat",
                                  "route_neginf", "route_n7k3", "route_allequal"])
def test_route_golden(name):
    lg, k = cases.route_cases()[name]
    idx, w = O.moe_route(lg, k)
    assert np.array_equal(idx, G[name + "_idx"])
    assert np.array_equal(bits(w), bits(G[name + "_w"]))


def test_route_kat_small():
    """qw6.c:3400-3412: logits {0,2,1,-1}, k=2 -> {1,2}, weights sum to 1."""
    idx, w = O.moe_route(np.array([0, 2, 1, -1], np.float32), 2)
    assert list(idx) == [1, 2] and abs(w.sum() - 1) < 1e-6 and w[0] > w[1]


def test_route_nan_kats():
    for lg, k, want in cases.nan_route_cases():
        lg = np.array(lg, np.float32)
        idx, w = O.moe_route(lg, k)
        assert list(idx) == want, (lg, idx, want)
        if np.isnan(lg[0]):
            assert np.isnan(w).all()   # qw6's max and softmax then propagate the NaN
        if O.ref() is not None:
            ri, rw = O.ref_moe_route(lg, k)
            assert np.array_equal(ri, idx)
            assert np.array_equal(bits(rw), bits(w))


def test_route_vectors_of_the_layer_tests():
    """The 256-expert routing vectors the layer-level GPU tests send through
    qw6_hip_moe_forward: the oracle's selections follow qw6's rules, worked
    by hand where the vector fixes them (an expert picked again once only
    -inf / NaN is left is index 0), and equal qw6's own build where present."""
    want = {n: list(O.moe_route(v, 8)[0]) for n, v in cases.route_vectors()}
    vec = dict(cases.route_vectors())
    assert want["allnan"] == [0] * 8
    assert want["allneginf"] == [0] * 8
    assert want["small_neginf"] == [1, 2, 0, 3, 0, 0, 0, 0]
    assert want["three_finite"] == [100, 200, 5, 0, 0, 0, 0, 0]
    assert want["allequal"] == list(range(8))
    assert want["nan_at_0"][0] == 0 and 0 not in want["nan_at_0"][1:]
    assert not set(want["nan_scattered"]) & {3, 17, 64, 65, 200, 255}
    assert sorted(want["low_index0"][:7]) == [0, 250, 251, 252, 253, 254, 255]
    assert want["low_index0"][7] == 0
    for i, (lg, _, hand) in enumerate(cases.nan_route_cases()):
        # padding with NaN keeps the hand-worked answer as the first ranks;
        # no later rank is a NaN's index
        got = want["nan%d" % i]
        assert got[:len(hand)] == hand
        assert all(k == 0 or not np.isnan(np.float32(lg[k])) for k in got)
    for n, v in vec.items():
        w = O.moe_route(v, 8)[1]
        if np.isnan(v[0]) or np.isneginf(v).all():
            assert np.isnan(w).all(), n   # the max is NaN, or -inf - -inf
        elif n in ("small_neginf", "three_finite", "low_index0"):
            assert np.isfinite(w).all() and w.sum() == pytest.approx(1.0, abs=1e-6), n
            rep = [k for k in range(8) if want[n][k] == 0][1:]   # index 0 again
            assert all(w[k] == 0.0 for k in rep), n
        if O.ref() is not None:
            ri, rw = O.ref_moe_route(v, 8)
            assert list(ri) == want[n], n
            assert np.array_equal(bits(rw), bits(w)), n


def test_route_brute_force_ties():
    """Top-k = stable argsort by (-value, index) on tiny inputs with duplicates."""
    rng = np.random.default_rng(3)
    for _ in range(300):
        n = int(rng.integers(2, 12))
        k = int(rng.integers(1, n + 1))
        lg = rng.integers(-3, 3, n).astype(np.float32)
        idx, w = O.moe_route(lg, min(k, 8))
        want = sorted(range(n), key=lambda i: (-lg[i], i))[:min(k, 8)]
        assert list(idx) == want
        e = np.exp(lg[want].astype(np.float64) - lg[want].max())
        assert np.allclose(w, e / e.sum(), atol=1e-6)


def test_rmsnorm_golden_and_kat():
    x = S.f32_normal(7, S.stream_id(0, S.K_X, 99), 2048, 1.0)
    assert np.array_equal(bits(O.rmsnorm(x, cases.norm_w(7, 0))), bits(G["rms_out"]))
    xk = np.array([1, -2, 3, -4], np.float32)   # qw6.c:3210-3223
    wk = np.array([1, 0.5, 2, -1], np.float32)
    sc = 1 / np.sqrt(np.float32(7.5) + np.float32(1e-6))
    assert np.abs(O.rmsnorm(xk, wk) - xk * sc * wk).max() < 1e-6


def test_silu_gather_kat():
    """qw6_vk.c:1789-1808 (silu_mul, n=513) and 1922-1954 (gather, dim 257)."""
    i = np.arange(513)
    g = (((i % 31).astype(np.float32) - 15) * 0.125).astype(np.float32)
    u = np.cos(i.astype(np.float32) * np.float32(0.031)).astype(np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.abs(O.silu_mul(g, u) - want).max() < 2e-5
    dim, k = 257, 8
    wts = (0.1 + 0.03 * np.arange(k)).astype(np.float32)
    wts /= wts.sum()
    e_, i_ = np.meshgrid(np.arange(k), np.arange(dim), indexing="ij")
    eo = np.sin((e_ * 17 + i_).astype(np.float32) * np.float32(0.021)).astype(np.float32)
    sh = np.cos(np.arange(dim, dtype=np.float32) * np.float32(0.019)).astype(np.float32)
    want = 0.25 * sh + wts @ eo.astype(np.float64)
    assert np.abs(O.moe_gather(eo, wts, sh, 0.25) - want).max() < 2e-5


@pytest.mark.parametrize("key", ["q4k_s11", "q4k_s12", "q4k_s13_noshared", "iq2m_s21", "iq2m_s22",
                                 "q4k_s14_sr", "iq2m_s23_sr"])
def test_layer_golden(key):
    """One layer, bit-exact against qw6_apply_layer_moe's outputs; the _sr
    cases weight the shared expert by sigmoid(shared_router . x)."""
    mix, rest = key.split("_", 1)
    seed = int(rest.split("_")[0][1:])
    shared = "noshared" not in rest
    L = cases.HostLayer(seed, 0, mix, shared=shared, shared_router=rest.endswith("_sr"))
    out, idx, w = cases.oracle_layer_out(L, cases.token_x(seed, 0))
    gk = "layer_" + key
    assert np.array_equal(idx, G[gk + "_idx"])
    assert np.array_equal(bits(w), bits(G[gk + "_w"]))
    assert np.array_equal(bits(out), bits(G[gk + "_out"]))


def test_stack_golden():
    seed = 41
    layers = [cases.HostLayer(seed, l, "iq2m") for l in range(3)]
    for step in range(2):
        h = cases.token_x(seed, 100, step)
        for l, L in enumerate(layers):
            xn = O.rmsnorm(h, cases.norm_w(seed, l))
            out, idx, _ = cases.oracle_layer_out(L, xn)
            assert np.array_equal(idx, G["stack_s%d_l%d_idx" % (step, l)])
            h = (h + out).astype(np.float32)
        assert np.array_equal(bits(h), bits(G["stack_s%d_h" % step]))


def test_prefill_given_logits_golden():
    seed = 51
    L = cases.HostLayer(seed, 0, "q4k")
    lg = S.zipf_logits(seed, 4)
    for t in range(4):
        out, idx, w = cases.oracle_layer_out(L, cases.token_x(seed, 0, t), logits=lg[t])
        assert np.array_equal(idx, G["prefill_t%d_idx" % t])
        assert np.array_equal(bits(out), bits(G["prefill_t%d_out" % t]))


@pytest.mark.skipif(O.ref() is None, reason="reference tree not built here")
@pytest.mark.parametrize("q", FORMATS)
def test_oracle_vs_reference_build_random(q):
    """Direct comparison with qw6's compiled CPU path on fresh seeds."""
    for seed in (101, 102):
        rows, cols = 12, 768
        w = S.quant_matrix(seed, 9, q, rows, cols)
        x = S.f32_normal(seed, 10, cols, 1.0)
        assert np.array_equal(bits(O.matvec(q, w, rows, cols, x)),
                              bits(O.ref_matvec(q, w, rows, cols, x)))


def test_planted_mistakes_are_caught():
    """A dropped term / wrong index in a restatement must fail the golden
    comparison: perturb one oracle output bit and one routing index."""
    w = S.quant_matrix(1, S.stream_id(0, S.K_GATE), S.Q_Q4_K_M, 512, 2048)
    x = S.f32_normal(1, S.stream_id(0, S.K_X), 2048, 1.0)
    y = O.matvec(S.Q_Q4_K_M, w, 512, 2048, x)
    y2 = y.copy()
    y2[17] = np.nextafter(y2[17], np.float32(np.inf))
    assert not np.array_equal(bits(y2), bits(G["cfg0_y"]))
    # a matvec with the high-nibble scale of sub-block 1 dropped differs
    w2 = w.copy().reshape(512, 8, 144)
    w2[:, :, 5] &= 0xC0
    assert not np.array_equal(bits(O.matvec(S.Q_Q4_K_M, w2.reshape(-1), 512, 2048, x)),
                              bits(G["cfg0_y"]))


# ---- greedy argmax (qw6_cpu_argmax, qw6.c:2858-2863) -------------------------------

def test_argmax_special_cases_and_selftest_kat():
    for x, want in cases.argmax_cases():
        assert O.argmax(np.array(x, np.float32)) == want, x


def test_argmax_brute_force_vs_numpy():
    """NaN-free inputs: numpy's argmax also returns the first maximum."""
    rng = np.random.default_rng(7)
    for n in (1, 2, 3, 17, 1000, 4099):
        for trial in range(20):
            x = rng.integers(-5, 6, n).astype(np.float32)   # many ties
            assert O.argmax(x) == int(np.argmax(x)), (n, trial)
            y = rng.standard_normal(n).astype(np.float32)
            assert O.argmax(y) == int(np.argmax(y))


@pytest.mark.skipif(O.ref() is None, reason="reference tree not built here")
def test_argmax_vs_reference_build():
    """Bitwise the reference's own function on random vectors with planted
    ties, NaNs, infinities and signed zeros."""
    rng = np.random.default_rng(11)
    R = O.ref()
    for x, _ in cases.argmax_cases():
        a = np.array(x, np.float32)
        assert O.argmax(a) == R.qw6_cpu_argmax(a, a.size)
    for n in (1, 5, 257, 248320):
        for trial in range(8):
            x = rng.standard_normal(n).astype(np.float32)
            k = rng.integers(0, n, size=min(n, 6))
            x[k[: len(k) // 2]] = x.max()                      # ties with the maximum
            x[k[len(k) // 2:]] = [np.nan, np.inf, -np.inf, -0.0, 0.0, np.nan][: len(k) - len(k) // 2]
            if trial == 0:
                x[0] = np.nan
            assert O.argmax(x) == R.qw6_cpu_argmax(x, n), (n, trial)


def test_argmax_planted_mistake_is_caught():
    """'>=' instead of '>' (last of the ties) or a reduction that lets a NaN
    win would fail the special cases above."""
    def last_tie(x):
        best = 0
        for i in range(1, len(x)):
            if x[i] >= x[best]:
                best = i
        return best
    def nan_wins(x):
        return int(np.argmax(np.array(x, np.float32)))   # numpy takes the first NaN
    cases_ = cases.argmax_cases()
    assert any(last_tie(np.array(x, np.float32)) != want for x, want in cases_)
    assert any(nan_wins(x) != want for x, want in cases_)
