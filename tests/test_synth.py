"""The seeded generator: determinism, layouts and distributions."""
import numpy as np

from qw6_amd import synth as S


def test_deterministic_and_sliceable():
    a = S.quant_blocks(5, 7, S.Q_Q4_K_M, 10)
    b = S.quant_blocks(5, 7, S.Q_Q4_K_M, 4, start=6)
    assert np.array_equal(a[6:], b)
    assert not np.array_equal(a, S.quant_blocks(6, 7, S.Q_Q4_K_M, 10))
    assert np.array_equal(S.rand_bytes(3, 4, 100)[40:], S.rand_bytes(3, 4, 60, start=40))


def test_scale_fields_distribution():
    blk = S.quant_blocks(9, 1, S.Q_Q4_K_M, 20000)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    assert (d >= 0).all()
    # |N(0,1)| * 2e-3: mean sqrt(2/pi) * 2e-3, a few percent fp16-subnormal
    assert abs(d.mean() / (np.sqrt(2 / np.pi) * 2e-3) - 1) < 0.02
    sub = (d < 2.0 ** -14).mean()
    assert 0.01 < sub < 0.04
    q6 = S.quant_blocks(9, 2, S.Q_Q6_K, 1000)
    d6 = q6[:, 208:210].copy().view(np.float16).astype(np.float32)
    assert abs(d6.mean() / (np.sqrt(2 / np.pi) * 1e-3) - 1) < 0.05


def test_normals_moments():
    z = S.normals(1, 2, 200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert np.abs(z).max() <= 6.0


def test_zipf_logits_topk_skew():
    lg = S.zipf_logits(3, 512)
    top = np.argsort(-lg, axis=1, kind="stable")[:, :8]
    counts = np.bincount(top.ravel(), minlength=256)
    assert counts.sum() == 512 * 8
    assert counts.max() > 5 * np.median(counts[counts > 0])
