"""Pin the CPU oracle (oracle/ring_attn_oracle.py) against things that are
fixed independently of it: a library routine (F.scaled_dot_product_attention
in fp64), fp64 autograd, brute-force loops, finite differences, and exact
identities of softmax attention.  The reference ships no tests or golden
vectors for this path, so these checks are what make the oracle trustworthy.
A last group plants mistakes in copies of the oracle math and shows the
checks reject them."""

import itertools
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import ring_attn_oracle as orc


def _inputs(B, H, T, D, N, seed=0, tc=None, scale_v=1.0):
    return orc.make_inputs(B, H, T, D, N, seed=seed, value_scale=scale_v, chunk_len=tc)


def _sdpa(q, k, v, mask=None):
    """fp64 SDPA on bf16-valued inputs; mask = boolean key mask [B, L] (True = keep)."""
    am = None if mask is None else mask[:, None, None, :]
    return F.scaled_dot_product_attention(q.double(), k.double(), v.double(), attn_mask=am)


def _lse(q, k, scale, mask=None):
    s = scale * torch.matmul(q.double(), k.double().transpose(-1, -2))
    if mask is not None:
        s = s.masked_fill(~mask[:, None, None, :], -math.inf)
    return torch.logsumexp(s, dim=-1, keepdim=True)


@pytest.mark.parametrize("D,N,T", [(64, 1, 64), (64, 4, 32), (72, 2, 48), (128, 3, 40)])
def test_forward_matches_sdpa(D, N, T):
    q, ks, vs, _ = _inputs(1, 2, T, D, N, seed=D + N)
    scale = 1.0 / math.sqrt(D)
    o, m, l = orc.ring_forward(q, ks, vs, scale)
    k = torch.cat(ks, dim=2)
    v = torch.cat(vs, dim=2)
    ref = _sdpa(q, k, v)
    assert torch.allclose(o, ref, atol=1e-12, rtol=1e-10)
    assert torch.allclose(orc.lse_from_ml(m, l), _lse(q, k, scale), atol=1e-12, rtol=1e-12)


def test_forward_masked_matches_sdpa_and_unpadded():
    B, H, T, D, N, tc = 2, 2, 24, 64, 3, 40
    lens = [40, 17, 33]
    q, ks, vs, _ = _inputs(B, H, T, D, N, seed=7, tc=tc)
    scale = 1.0 / math.sqrt(D)
    o, m, l = orc.ring_forward(q, ks, vs, scale, kv_valid_lens=lens)
    k = torch.cat(ks, dim=2)
    v = torch.cat(vs, dim=2)
    mask = torch.zeros(B, N * tc, dtype=torch.bool)
    for c, n in enumerate(lens):
        mask[:, c * tc: c * tc + n] = True
    assert torch.allclose(o, _sdpa(q, k, v, mask), atol=1e-12)
    assert torch.allclose(orc.lse_from_ml(m, l), _lse(q, k, scale, mask), atol=1e-12)
    # padded + masked == the unpadded problem
    ks_u = [kc[:, :, :n] for kc, n in zip(ks, lens)]
    vs_u = [vc[:, :, :n] for vc, n in zip(vs, lens)]
    o2, m2, l2 = orc.ring_forward(q, ks_u, vs_u, scale)
    assert torch.allclose(o, o2, atol=1e-13)


def test_forward_bruteforce_tiny():
    q, ks, vs, _ = _inputs(1, 1, 3, 8, 2, seed=3, tc=3)
    scale = 0.37
    o, m, l = orc.ring_forward(q, ks, vs, scale)
    keys = [kc[0, 0, j] for kc in ks for j in range(kc.shape[2])]
    vals = [vc[0, 0, j] for vc in vs for j in range(vc.shape[2])]
    for i in range(3):
        qi = q[0, 0, i].double()
        sc = [scale * sum(float(qi[d]) * float(kk[d]) for d in range(8)) for kk in keys]
        mx = max(sc)
        w = [math.exp(s - mx) for s in sc]
        z = sum(w)
        out = [sum(w[j] * float(vals[j][d]) for j in range(len(w))) / z for d in range(8)]
        assert max(abs(out[d] - float(o[0, 0, i, d])) for d in range(8)) < 1e-12
        assert abs((mx + math.log(z)) - float(orc.lse_from_ml(m, l)[0, 0, i, 0])) < 1e-12


@pytest.mark.parametrize("N", [2, 4, 8])
def test_ring_rank_and_order_invariance(N):
    q, ks, vs, _ = _inputs(1, 2, 16, 64, N, seed=N)
    scale = 0.125
    o0, m0, l0 = orc.ring_forward(q, ks, vs, scale, ring_rank=0)
    lse0 = orc.lse_from_ml(m0, l0)
    for r in range(1, N):
        o, m, l = orc.ring_forward(q, ks, vs, scale, ring_rank=r)
        assert torch.allclose(o, o0, atol=1e-13)
        assert torch.allclose(orc.lse_from_ml(m, l), lse0, atol=1e-13)
    perm = list(reversed(range(N)))
    o, m, l = orc.ring_forward(q, [ks[i] for i in perm], [vs[i] for i in perm], scale)
    assert torch.allclose(o, o0, atol=1e-13)


def test_lse_associativity_and_single_chunk_reduction():
    q, ks, vs, _ = _inputs(1, 2, 16, 64, 2, seed=11)
    scale = 0.125
    _, ma, la = orc.ring_forward(q, ks[:1], vs[:1], scale)
    _, mb, lb = orc.ring_forward(q, ks[1:], vs[1:], scale)
    _, m, l = orc.ring_forward(q, ks, vs, scale)
    lhs = orc.lse_from_ml(m, l)
    rhs = torch.logaddexp(orc.lse_from_ml(ma, la), orc.lse_from_ml(mb, lb))
    assert torch.allclose(lhs, rhs, atol=1e-13)
    # N = 1 is plain attention
    o1, _, _ = orc.ring_forward(q, ks[:1], vs[:1], scale)
    assert torch.allclose(o1, _sdpa(q, ks[0], vs[0]), atol=1e-12)


def _autograd_ref(q, ks, vs, do, scale, lens=None):
    k = torch.cat(ks, dim=2).double().requires_grad_(True)
    v = torch.cat(vs, dim=2).double().requires_grad_(True)
    qq = q.double().requires_grad_(True)
    mask = None
    if lens is not None:
        tc = ks[0].shape[2]
        mask = torch.zeros(q.shape[0], len(ks) * tc, dtype=torch.bool)
        for c, n in enumerate(lens):
            mask[:, c * tc: c * tc + n] = True
    am = None if mask is None else mask[:, None, None, :]
    o = F.scaled_dot_product_attention(qq, k, v, attn_mask=am, scale=scale)
    o.backward(do.double())
    return qq.grad, k.grad, v.grad


@pytest.mark.parametrize("D,N,lens", [(64, 1, None), (72, 2, None), (128, 4, None), (64, 3, [20, 7, 13])])
def test_backward_matches_autograd(D, N, lens):
    tc = 20 if lens else 24
    q, ks, vs, do = _inputs(1, 2, 24, D, N, seed=D * N, tc=tc)
    scale = 1.0 / math.sqrt(D)
    o, m, l = orc.ring_forward(q, ks, vs, scale, kv_valid_lens=lens)
    Dl = orc.delta(do, o)
    dq, dks, dvs = orc.ring_backward(q, ks, vs, do, m, l, Dl, scale, kv_valid_lens=lens)
    gq, gk, gv = _autograd_ref(q, ks, vs, do, scale, lens)
    assert torch.allclose(dq, gq, atol=1e-11)
    assert torch.allclose(torch.cat(dks, dim=2), gk, atol=1e-11)
    assert torch.allclose(torch.cat(dvs, dim=2), gv, atol=1e-11)


def test_backward_finite_differences():
    q, ks, vs, do = _inputs(1, 1, 4, 8, 2, seed=5, tc=3)
    q, ks, vs, do = q.double(), [k.double() for k in ks], [v.double() for v in vs], do.double()
    scale = 0.4
    o, m, l = orc.ring_forward(q, ks, vs, scale)
    dq, dks, dvs = orc.ring_backward(q, ks, vs, do, m, l, orc.delta(do, o), scale)

    def loss(qq, kk, vv):
        return float((orc.ring_forward(qq, kk, vv, scale)[0] * do).sum())

    eps = 1e-6
    for (i, d) in itertools.product(range(4), range(0, 8, 3)):
        qp, qm = q.clone(), q.clone()
        qp[0, 0, i, d] += eps
        qm[0, 0, i, d] -= eps
        fd = (loss(qp, ks, vs) - loss(qm, ks, vs)) / (2 * eps)
        assert abs(fd - float(dq[0, 0, i, d])) < 1e-7
    for c, j, d in itertools.product(range(2), range(3), (1, 6)):
        kp = [k.clone() for k in ks]
        km = [k.clone() for k in ks]
        kp[c][0, 0, j, d] += eps
        km[c][0, 0, j, d] -= eps
        fd = (loss(q, kp, vs) - loss(q, km, vs)) / (2 * eps)
        assert abs(fd - float(dks[c][0, 0, j, d])) < 1e-7
        vp = [v.clone() for v in vs]
        vm = [v.clone() for v in vs]
        vp[c][0, 0, j, d] += eps
        vm[c][0, 0, j, d] -= eps
        fd = (loss(q, ks, vp) - loss(q, ks, vm)) / (2 * eps)
        assert abs(fd - float(dvs[c][0, 0, j, d])) < 1e-7


def test_delta_identity_and_gradient_sums():
    q, ks, vs, do = _inputs(1, 2, 32, 64, 2, seed=9)
    scale = 0.125
    o, m, l = orc.ring_forward(q, ks, vs, scale)
    Dl = orc.delta(do, o)
    k = torch.cat(ks, dim=2).double()
    v = torch.cat(vs, dim=2).double()
    p = torch.softmax(scale * q.double() @ k.transpose(-1, -2), dim=-1)
    dp = do.double() @ v.transpose(-1, -2)
    assert torch.allclose(Dl, (p * dp).sum(-1, keepdim=True), atol=1e-12)
    dq, dks, dvs = orc.ring_backward(q, ks, vs, do, m, l, Dl, scale)
    dk = torch.cat(dks, dim=2)
    dv = torch.cat(dvs, dim=2)
    # sum_j dS_ij = 0  =>  sum over keys of dK = 0 ;  sum_j P_ij = 1  =>  sum over keys of dV = sum over queries of dO
    assert dk.sum(dim=2).abs().max() < 1e-10 * dk.abs().max() * dk.shape[2]
    assert torch.allclose(dv.sum(dim=2), do.double().sum(dim=2), atol=1e-10)


def test_reference_rounding_mode_is_close_but_distinct():
    q, ks, vs, _ = _inputs(1, 2, 32, 128, 2, seed=2)
    scale = 1.0 / math.sqrt(128)
    o, _, _ = orc.ring_forward(q, ks, vs, scale)
    o_r, m_r, _ = orc.ring_forward(q, ks, vs, scale, reference_rounding=True)
    err = (o_r - o).norm() / o.norm()
    assert 0 < err < 2e-2  # the reference's own truncations stay within the parity bar
    assert torch.equal(m_r, m_r.to(torch.bfloat16).double())


# --- planted mistakes: each must be caught by one of the checks above -------

def _forward_variant(q, ks, vs, scale, bug):
    B, H, T, D = q.shape
    m = torch.full((B, H, T, 1), -math.inf, dtype=torch.float64)
    l = torch.zeros((B, H, T, 1), dtype=torch.float64)
    o = torch.zeros((B, H, T, D), dtype=torch.float64)
    for kc, vc in zip(ks, vs):
        s = scale * q.double() @ kc.double().transpose(-1, -2)
        m_new = torch.maximum(m, s.amax(-1, keepdim=True))
        corr = torch.exp(m - m_new)
        if bug == "no_corr_on_o":
            corr_o = torch.ones_like(corr)
        else:
            corr_o = corr
        p = torch.exp(s - m_new)
        if bug == "transposed_v":
            p_v = p @ vc.double().flip(-2)
        else:
            p_v = p @ vc.double()
        l = l * corr + p.sum(-1, keepdim=True)
        o = o * corr_o + p_v
        m = m_new
    return o / l


@pytest.mark.parametrize("bug", ["no_corr_on_o", "transposed_v"])
def test_planted_forward_mistakes_are_caught(bug):
    q, ks, vs, _ = _inputs(1, 2, 16, 64, 4, seed=1)
    scale = 0.125
    good = _forward_variant(q, ks, vs, scale, None)
    bad = _forward_variant(q, ks, vs, scale, bug)
    ref = _sdpa(q, torch.cat(ks, 2), torch.cat(vs, 2))
    assert torch.allclose(good, ref, atol=1e-12)
    assert (bad - ref).norm() / ref.norm() > 2e-2


def test_planted_backward_sign_mistake_is_caught():
    q, ks, vs, do = _inputs(1, 2, 24, 64, 2, seed=4)
    scale = 0.125
    o, m, l = orc.ring_forward(q, ks, vs, scale)
    # wrong sign of D in dS: dS = P (dP + D) scale
    _, dks, _ = orc.ring_backward(q, ks, vs, do, m, l, -orc.delta(do, o), scale)
    _, gk, _ = _autograd_ref(q, ks, vs, do, scale)
    assert (torch.cat(dks, 2) - gk).norm() / gk.norm() > 3e-2
