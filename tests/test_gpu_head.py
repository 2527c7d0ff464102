"""The greedy next-token head on the GPU (qw6_hip_argmax, qw6_hip_argmax_host,
qw6_hip_output_greedy) against the oracle, through the C ABI.

argmax: bit-exact with qw6_cpu_argmax's rule on random vectors with planted
ties, NaNs, infinities and signed zeros, up to and past the 248,320-entry
vocabulary. Output head: logits rel-L2 <= 1e-5 against the oracle's RMSNorm
and matvec; the token equals the argmax of the GPU's own logits exactly, and
the oracle's token unless the top two oracle logits are closer than 1e-4
relative (the GPU sums each row in another order).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import cases
import oracle as O
import qw6_amd as Q
from qw6_amd import synth as S

pytestmark = pytest.mark.gpu

TOL = 1e-5
TIE = 1e-4
HIDDEN = 2048
VOCAB = 248320


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "no GPU visible"
    return torch


@pytest.fixture(scope="module")
def ctx(torch_dev):
    c = Q.Context(0, max_tokens=1)
    yield c
    c.close()


def planted(rng, n, trial):
    x = rng.standard_normal(n).astype(np.float32)
    k = rng.integers(0, n, size=min(n, 6))
    x[k[: len(k) // 2]] = x.max()
    x[k[len(k) // 2:]] = [np.nan, np.inf, -np.inf, -0.0, 0.0, np.nan][: len(k) - len(k) // 2]
    if trial == 1:
        x[0] = np.nan
    if trial == 2:
        x[:] = np.round(x)   # many ties
    return x


def dev_argmax(torch, ctx, x, offset=0):
    buf = torch.from_numpy(np.concatenate([np.zeros(offset, np.float32), x])).cuda()
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.argmax(buf.data_ptr() + 4 * offset, x.size, out)
    torch.cuda.synchronize()
    return int(out.cpu().numpy().view(np.uint32)[0])


def test_argmax_device_and_host_vs_oracle(torch_dev, ctx):
    rng = np.random.default_rng(21)
    vecs = [np.array(x, np.float32) for x, _ in cases.argmax_cases()]
    for n in (1, 2, 3, 5, 1000, 1023, 1024, 1025, 4097, 65537, VOCAB, 1 << 21):
        for trial in range(3):
            vecs.append(planted(rng, n, trial))
    for i, x in enumerate(vecs):
        want = O.argmax(x)
        assert dev_argmax(torch_dev, ctx, x) == want, (i, x.size)
        if x.size <= 65537:
            got, val = Q.argmax_host(x, with_value=True)
            assert got == want, (i, x.size)
            assert np.array_equal(np.float32(val).view(np.uint32), x[want].view(np.uint32))
            assert Q.sampling_greedy_host(x) == want, (i, x.size)
    say("argmax vectors checked:", len(vecs))


def test_host_argmax_and_greedy_kats():
    """qw6's Vulkan self-test vectors for the two host ops (qw6_vk.c:1810-1838):
    argmax over 4097 values with 42 planted at 3079 (index and value), and
    greedy sampling over 1029 logits with 11 planted at 877."""
    an = 4097
    i = np.arange(an, dtype=np.float32)
    ax = (np.sin(i * np.float32(0.019)) - (np.arange(an) % 7).astype(np.float32) * np.float32(0.01)
          ).astype(np.float32)
    ax[3079] = 42.0
    assert Q.argmax_host(ax, with_value=True) == (3079, np.float32(42.0))
    gn = 1029
    j = np.arange(gn, dtype=np.float32)
    gx = (np.cos(j * np.float32(0.023)) - np.float32(0.001) * j).astype(np.float32)
    gx[877] = 11.0
    assert Q.sampling_greedy_host(gx) == 877
    with pytest.raises(Q.Qw6HipError):
        Q.sampling_greedy_host(np.zeros(0, np.float32))


def test_argmax_unaligned_and_ties_across_blocks(torch_dev, ctx):
    """A start that is not 16-byte aligned (the scalar path), and equal maxima
    that land in different first-pass blocks: the lowest index wins."""
    rng = np.random.default_rng(22)
    for n in (7, 4097, VOCAB):
        x = rng.standard_normal(n).astype(np.float32)
        for off in (1, 2, 3):
            assert dev_argmax(torch_dev, ctx, x, offset=off) == O.argmax(x), (n, off)
    x = rng.standard_normal(VOCAB).astype(np.float32)
    m = np.float32(x.max() + 1)
    for i in (200000, 5000, 1100, 4):
        x[i] = m
    assert dev_argmax(torch_dev, ctx, x) == 4 == O.argmax(x)
    x[4] = np.nan   # a NaN away from index 0 is skipped
    assert dev_argmax(torch_dev, ctx, x) == 1100 == O.argmax(x)


def run_head(torch, ctx, w_dev, q, rows, x, nw):
    dx = torch.from_numpy(x).cuda()
    dn = None if nw is None else torch.from_numpy(nw).cuda()
    logits = torch.zeros(rows, dtype=torch.float32, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.output_greedy((w_dev, q, rows, HIDDEN), dx, logits, tok, norm_w=dn, eps=1e-6)
    torch.cuda.synchronize()
    return logits.cpu().numpy(), int(tok.cpu().numpy().view(np.uint32)[0])


@pytest.mark.parametrize("q", [S.Q_Q6_K, S.Q_Q4_K_M, S.Q_IQ2_XXS, S.Q_FP32])
@pytest.mark.parametrize("with_norm", [True, False])
def test_output_greedy_vs_oracle(torch_dev, ctx, q, with_norm):
    torch = torch_dev
    vocab = 4096
    say("output head", q, with_norm)
    if q == S.Q_FP32:
        w = S.f32_normal(31, S.stream_id(0, S.K_OUTPUT), vocab * HIDDEN, 0.02)
    else:
        w = S.quant_matrix(31, S.stream_id(0, S.K_OUTPUT), q, vocab, HIDDEN)
    dw = torch.from_numpy(np.ascontiguousarray(w).view(np.uint8)).cuda()
    x = cases.token_x(32, 0)
    nw = S.f32_normal(33, S.stream_id(0, S.K_ONORM), HIDDEN, 0.1, mean=1.0) if with_norm else None
    glog, gtok = run_head(torch, ctx, dw.data_ptr(), q, vocab, x, nw)
    xn = O.rmsnorm(x, nw, 1e-6) if with_norm else x
    olog = O.matvec(q, w, vocab, HIDDEN, xn)
    assert cases.rel_l2(glog, olog) <= TOL
    assert gtok == O.argmax(glog)
    s = np.sort(olog)[-2:]
    if s[1] - s[0] > TIE * max(abs(float(s[1])), 1e-30):
        assert gtok == O.argmax(olog)
    else:
        say("near tie in the oracle logits, token compared with the GPU logits only")


def test_output_greedy_full_vocab(torch_dev, ctx):
    """Q6_K [248320 x 2048] (417 MB) generated on the device: the token is the
    exact argmax of the returned logits, and 64 random rows match the oracle."""
    torch = torch_dev
    q = S.Q_Q6_K
    rb = S.row_bytes(q, HIDDEN)
    w = torch.empty(VOCAB * rb, dtype=torch.uint8, device="cuda")
    Q.synth_blocks(w, q, VOCAB * HIDDEN // 256, 34, S.stream_id(0, S.K_OUTPUT))
    x = cases.token_x(35, 0)
    nw = S.f32_normal(36, S.stream_id(0, S.K_ONORM), HIDDEN, 0.1, mean=1.0)
    glog, gtok = run_head(torch, ctx, w.data_ptr(), q, VOCAB, x, nw)
    assert gtok == O.argmax(glog)
    rows = np.random.default_rng(37).choice(VOCAB, 64, replace=False)
    xn = O.rmsnorm(x, nw, 1e-6)
    nb = HIDDEN // 256
    want = np.array([O.matvec(q, S.quant_blocks(34, S.stream_id(0, S.K_OUTPUT), q, nb, start=int(r) * nb),
                              1, HIDDEN, xn)[0] for r in rows], np.float32)
    assert cases.rel_l2(glog[rows], want) <= TOL
    say("full-vocab token", gtok)


@pytest.mark.parametrize("hidden,rows", [(256, 1024), (1024, 777), (1024, 2000), (512, 3001)])
def test_output_greedy_other_shapes(torch_dev, ctx, hidden, rows):
    """Rows of 256 / 512 / 1024 columns (8, 4, 2 rows per wave step), and row
    counts that are not a multiple of a step (those take the plain matvec
    and the two-pass argmax): logits and token against the oracle."""
    torch = torch_dev
    q = S.Q_Q6_K
    w = S.quant_matrix(41, S.stream_id(1, S.K_OUTPUT), q, rows, hidden)
    dw = torch.from_numpy(w).cuda()
    x = S.f32_normal(42, S.stream_id(1, S.K_X), hidden, 1.0)
    nw = S.f32_normal(43, S.stream_id(1, S.K_ONORM), hidden, 0.1, mean=1.0)
    dx, dn = torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda()
    logits = torch.zeros(rows, dtype=torch.float32, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.output_greedy((dw.data_ptr(), q, rows, hidden), dx, logits, tok, norm_w=dn, eps=1e-6)
    torch.cuda.synchronize()
    glog = logits.cpu().numpy()
    gtok = int(tok.cpu().numpy().view(np.uint32)[0])
    olog = O.matvec(q, w, rows, hidden, O.rmsnorm(x, nw, 1e-6))
    assert cases.rel_l2(glog, olog) <= TOL
    assert gtok == O.argmax(glog)


@pytest.mark.parametrize("rows,offset", [(4008, 0), (4096, 2), (1600, 0)])
def test_output_greedy_q6k_2048_dispatch(torch_dev, ctx, rows, offset):
    """Q6_K rows of 2048 columns either side of the bf16-MFMA head's
    conditions: 4008 rows (not a multiple of its 16-row tiles) take the fp32
    kernel, 1600 rows (100 tiles, a small grid) the MFMA kernel; logits and
    token against the oracle. Weight data 2 bytes past 16-byte alignment is
    refused before any launch (the matrix contract)."""
    torch = torch_dev
    q = S.Q_Q6_K
    w = S.quant_matrix(44, S.stream_id(2, S.K_OUTPUT), q, rows, HIDDEN)
    buf = torch.zeros(w.nbytes + 16, dtype=torch.uint8, device="cuda")
    buf[offset:offset + w.nbytes] = torch.from_numpy(np.ascontiguousarray(w).view(np.uint8)).cuda()
    x = cases.token_x(45, 0)
    nw = S.f32_normal(46, S.stream_id(2, S.K_ONORM), HIDDEN, 0.1, mean=1.0)
    dx, dn = torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda()
    logits = torch.zeros(rows, dtype=torch.float32, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    if offset % 16:
        with pytest.raises(Q.Qw6HipError, match="aligned"):
            ctx.output_greedy((buf.data_ptr() + offset, q, rows, HIDDEN), dx, logits, tok, norm_w=dn, eps=1e-6)
        return
    ctx.output_greedy((buf.data_ptr() + offset, q, rows, HIDDEN), dx, logits, tok, norm_w=dn, eps=1e-6)
    torch.cuda.synchronize()
    glog = logits.cpu().numpy()
    gtok = int(tok.cpu().numpy().view(np.uint32)[0])
    olog = O.matvec(q, w, rows, HIDDEN, O.rmsnorm(x, nw, 1e-6))
    rel = cases.rel_l2(glog, olog)
    say("Q6_K x 2048, %d rows, offset %d: rel-L2 %.2e" % (rows, offset, rel))
    assert rel <= TOL
    assert gtok == O.argmax(glog)

