"""Pins of oracle/h3_ref.py (the H3 per-segment transforms) on the CPU.

Golden cases from the reference's own camera tests (test_camera.py:50-100), the algebra the
camera matrices must satisfy, rotation properties of the rotary part and bit-exact special
cases of the bf16 chain.
"""

import math

import pytest
import torch

from oracle import h3_ref as h3
from oracle import prope_ref as pr
from oracle import segments_ref as sr

BF = torch.bfloat16


def _rotation(g, n, dtype=torch.float64):
    a = torch.randn(n, 3, 3, generator=g, dtype=torch.float64)
    qm, r = torch.linalg.qr(a)
    qm = qm * torch.sign(torch.diagonal(r, dim1=-2, dim2=-1))[:, None, :]
    det = torch.linalg.det(qm)
    qm[det < 0, :, 0] *= -1
    return qm.to(dtype)


def _poses(g, n, dtype=torch.float64, t_scale=2.0):
    m = torch.zeros(n, 4, 4, dtype=torch.float64)
    m[:, :3, :3] = _rotation(g, n)
    m[:, :3, 3] = torch.randn(n, 3, generator=g, dtype=torch.float64) * t_scale
    m[:, 3, 3] = 1.0
    return m.to(dtype)


def _intrinsics(n, focal=1.0):
    k = torch.eye(3, dtype=torch.float64).repeat(n, 1, 1)
    k[:, 0, 0] = k[:, 1, 1] = focal
    k[:, 0, 2] = k[:, 1, 2] = 0.5
    return k


def test_logd4_golden_case():
    """test_camera.py:50-56: t = (3, 4, 0) -> t log1p(5) / 20; t = 0 stays 0."""
    v = torch.eye(4, dtype=torch.float64).repeat(2, 1, 1)
    v[1, :3, 3] = torch.tensor([3.0, 4.0, 0.0], dtype=torch.float64)
    out = pr.transform_relative_viewmats(v, "logd4")
    assert torch.equal(out[0, :3, 3], torch.zeros(3, dtype=torch.float64))
    want = torch.tensor([3.0, 4.0, 0.0], dtype=torch.float64) * math.log1p(5.0) / 20.0
    torch.testing.assert_close(out[1, :3, 3], want, rtol=1e-14, atol=0)
    assert torch.equal(out[..., :3, :3], v[..., :3, :3])


def test_fixed_focal_ignores_input_intrinsics():
    """test_camera.py:94-100: matrices from intrinsics of focal 0.7 and 1.7 are equal."""
    g = torch.Generator().manual_seed(1)
    v = _poses(g, 3)
    a = h3.suffix_matrices(v, _intrinsics(3, 0.7))
    b = h3.suffix_matrices(v, _intrinsics(3, 1.7))
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    p = a[2]
    assert p[0, 0, 0] != 0 and abs(float(p[..., 0, :3].norm(dim=-1)[0]) - h3.WAN_FIXED_FX) < 1e-12


def test_camera_matrices_invert_and_keep_inner_products():
    """P⁻¹ P = I; Pᵀ q and P⁻¹ k keep every 4-vector inner product for one camera and the output
    map undoes the value map (test_camera.py:59-80), through the bf16 projection kernel's
    restatement (bf16 tolerance)."""
    g = torch.Generator().manual_seed(2)
    n = 6
    v = pr.transform_relative_viewmats(_poses(g, n), "logd4")
    q_t, p_inv, p = h3.suffix_matrices(v, _intrinsics(n))
    eye = torch.eye(4, dtype=torch.float64).expand(n, 4, 4)
    torch.testing.assert_close(p_inv @ p, eye, rtol=0, atol=1e-12)
    torch.testing.assert_close(q_t, p.transpose(-1, -2), rtol=0, atol=0)
    x = torch.randn(1, n, 3, 128, generator=g).to(BF)
    y = torch.randn(1, n, 3, 128, generator=g).to(BF)
    qx = h3.prope_project(x, q_t[None].float())
    ky = h3.prope_project(y, p_inv[None].float())
    assert torch.equal(qx[..., :96], x[..., :96]) and torch.equal(ky[..., :96], y[..., :96])
    before = (x[..., 96:].double().reshape(1, n, 3, 8, 4) * y[..., 96:].double().reshape(1, n, 3, 8, 4)).sum(-1)
    after = (qx[..., 96:].double().reshape(1, n, 3, 8, 4) * ky[..., 96:].double().reshape(1, n, 3, 8, 4)).sum(-1)
    torch.testing.assert_close(after, before, rtol=0, atol=0.12)
    back = h3.prope_project(h3.prope_project(x, p_inv[None].float()), p[None].float())
    torch.testing.assert_close(back.double(), x.double(), rtol=0.03, atol=0.03)
    # a transposed query matrix breaks the pairing
    wrong = h3.prope_project(x, p[None].float())
    bad = (wrong[..., 96:].double().reshape(1, n, 3, 8, 4) * ky[..., 96:].double().reshape(1, n, 3, 8, 4)).sum(-1)
    assert float((bad - before).abs().max()) > 1.0


def test_scores_depend_on_the_relative_pose_only():
    """A rotation of the world frame applied to every camera (V -> V W, W a rotation, which
    keeps every translation and so logd4's scale) leaves q' . k' unchanged (float64)."""
    g = torch.Generator().manual_seed(3)
    n = 5
    v = _poses(g, n)
    w = torch.eye(4, dtype=torch.float64)
    w[:3, :3] = _rotation(g, 1)[0]
    qm, km, _ = h3.prope_qkv_separate_matrices(v, _intrinsics(n), v, _intrinsics(n), torch.float64)
    qm2, km2, _ = h3.prope_qkv_separate_matrices(v @ w, _intrinsics(n), v @ w, _intrinsics(n),
                                                  torch.float64)
    x = torch.randn(n, 4, dtype=torch.float64, generator=g)
    y = torch.randn(n, 4, dtype=torch.float64, generator=g)
    # all query/key camera pairs (i, j)
    qx = torch.einsum("iab,ib->ia", qm, x)
    ky = torch.einsum("jab,jb->ja", km, y)
    qx2 = torch.einsum("iab,ib->ia", qm2, x)
    ky2 = torch.einsum("jab,jb->ja", km2, y)
    torch.testing.assert_close(qx @ ky.T, qx2 @ ky2.T, rtol=1e-10, atol=1e-10)
    # and they do depend on the pose: a different key camera changes them
    v3 = v.clone()
    v3[0, :3, 3] += 1.0
    _, km3, _ = h3.prope_qkv_separate_matrices(v, _intrinsics(n), v3, _intrinsics(n), torch.float64)
    ky3 = torch.einsum("jab,jb->ja", km3, y)
    assert float((qx @ ky3.T - qx @ ky.T).abs().max()) > 1e-3


def _angles_tables(theta):
    """cos / sin [S, 96] with each pair (i, i + 48) turned by theta[:, i]."""
    c, s = torch.cos(theta), torch.sin(theta)
    return torch.cat([c, c], 1), torch.cat([s, s], 1)


def test_rotary_special_cases_are_bit_exact():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 7, 3, 128, generator=g).to(BF)
    ones, zeros = torch.ones(7, 96), torch.zeros(7, 96)
    eye = torch.eye(4).expand(1, 7, 4, 4)
    assert torch.equal(h3.rope_prope(x, ones, zeros, eye), x)
    y = h3.rope_prope(x, zeros, ones, None)
    assert torch.equal(y[..., :48], -x[..., 48:96]) and torch.equal(y[..., 48:96], x[..., :48])
    assert torch.equal(y[..., 96:], x[..., 96:])


def test_rotary_preserves_norms_and_composes():
    g = torch.Generator().manual_seed(5)
    S = 9
    x = torch.randn(1, S, 2, 128, generator=g).to(BF)
    a = torch.rand(S, 48, generator=g, dtype=torch.float64) * 6.0
    b = torch.rand(S, 48, generator=g, dtype=torch.float64) * 6.0
    ca, sa = _angles_tables(a)
    cb, sb = _angles_tables(b)
    cab, sab = _angles_tables(a + b)
    y = h3.rope_prope(x, ca, sa, None).double()
    xd = x.double()
    n0 = xd[..., :48] ** 2 + xd[..., 48:96] ** 2
    n1 = y[..., :48] ** 2 + y[..., 48:96] ** 2
    torch.testing.assert_close(n1, n0, rtol=0.04, atol=1e-3)
    two = h3.rope_prope(h3.rope_prope(x, ca, sa, None), cb, sb, None).double()
    one = h3.rope_prope(x, cab, sab, None).double()
    torch.testing.assert_close(two[..., :96], one[..., :96], rtol=0, atol=0.06)
    # the rotation direction: a quarter turn maps (x1, x2) to (-x2, x1), not (x2, -x1)
    q = torch.full((S, 48), math.pi / 2, dtype=torch.float64)
    cq, sq = _angles_tables(q)
    z = h3.rope_prope(x, cq, sq, None).double()
    torch.testing.assert_close(z[..., :48], -xd[..., 48:96], rtol=0.01, atol=0.01)


def test_projection_matches_float64_and_its_sum_order():
    g = torch.Generator().manual_seed(6)
    B, S, H = 2, 5, 3
    x = torch.randn(B, S, H, 128, generator=g).to(BF)
    m = (torch.randn(B, S, 4, 4, generator=g) * 0.7).to(BF)
    y = h3.prope_project(x, m)
    xs = x[..., 96:].double().reshape(B, S, H, 8, 4)
    gold = torch.einsum("bsij,bshpj->bshpi", m.double(), xs)
    terms = torch.einsum("bsij,bshpj->bshpi", m.double().abs(), xs.abs())
    err = (y[..., 96:].double().reshape(B, S, H, 8, 4) - gold).abs()
    assert bool((err <= 2.0 ** -8 * gold.abs() + 1e-6 * terms).all())  # one bf16 rounding
    assert torch.equal(y[..., :96], x[..., :96])
    # explicit per-element loop, same sum order
    for bb in range(B):
        for s in range(S):
            for h in range(H):
                for p in range(8):
                    v = [float(x[bb, s, h, 96 + 4 * p + j]) for j in range(4)]
                    for i in range(4):
                        mm = [float(m[bb, s, i, j]) for j in range(4)]
                        t = torch.tensor(mm[0] * v[0], dtype=torch.float32)
                        t = t + torch.tensor(mm[1] * v[1], dtype=torch.float32)
                        t = t + torch.tensor(mm[2] * v[2], dtype=torch.float32)
                        t = t + torch.tensor(mm[3] * v[3], dtype=torch.float32)
                        assert torch.equal(t.to(BF), y[bb, s, h, 96 + 4 * p + i]), (bb, s, h, p, i)


def test_identity_transforms_reduce_to_the_plain_window():
    g = torch.Generator().manual_seed(7)
    T, H, cf, P = 16, 2, 2, 20
    pk, pv = (torch.randn(1, P, H, 128, generator=g).to(BF) for _ in range(2))
    c1, c2 = sr.H3RawKVCache(), sr.H3RawKVCache()
    for c in range(3):
        q, k, v = (torch.randn(1, cf * T, H, 128, generator=g).to(BF) for _ in range(3))
        nk = P + (min(c, 5) + 1) * cf * T
        ones, zeros = torch.ones(nk, 96), torch.zeros(nk, 96)
        eye = torch.eye(4).expand(1, nk, 4, 4)
        got = h3.windowed_rollout_attention(
            q, k, v, pk, pv, c1, 0, c, q_rotary=(ones[: cf * T], zeros[: cf * T]),
            k_rotary=(ones, zeros), q_matrix=eye[:, : cf * T], kv_matrix=eye,
            out_matrix=eye[:, : cf * T], commit=True)
        want = sr.windowed_rollout_attention(q, k, v, pk, pv, c2, 0, c, commit=True)
        assert torch.equal(got, want.to(BF))


def test_memory_form_identity_and_per_segment_transforms():
    g = torch.Generator().manual_seed(8)
    T, H, text, n_bank, audio, C = 8, 2, 5, 2, 3, 16
    prefix = text + T + n_bank * T + audio
    L = prefix + C
    q, k, v = (torch.randn(1, L, H, 128, generator=g).to(BF) for _ in range(3))
    hk, hv = (torch.randn(1, 2 * C, H, 128, generator=g).to(BF) for _ in range(2))
    kw = dict(text_rows=text, frame_rows=T, n_bank=n_bank, audio_rows=audio)
    ones, zeros = torch.ones(L, 96), torch.zeros(L, 96)
    eye = torch.eye(4).expand(1, L, 4, 4)
    heye = torch.eye(4).expand(1, 2 * C, 4, 4)
    got = h3.memory_kv_attention(q, k, v, hk, hv, rotary=(ones, zeros),
                                 history_rotary=(ones[:2 * C], zeros[:2 * C]), q_matrix=eye,
                                 kv_matrix=eye, out_matrix=eye, history_kv_matrix=heye, **kw)
    assert torch.equal(got, sr.memory_kv_attention(q, k, v, hk, hv, **kw).to(BF))
    # per-segment transforms of the gathered rows (the reference's calculate) give the same
    cos, sin = (torch.randn(L, 96, generator=g) for _ in range(2))
    hc, hs = (torch.randn(2 * C, 96, generator=g) for _ in range(2))
    qm, km, om = (torch.randn(1, L, 4, 4, generator=g) * 0.5 for _ in range(3))
    hm = torch.randn(1, 2 * C, 4, 4, generator=g) * 0.5
    got = h3.memory_kv_attention(q, k, v, hk, hv, rotary=(cos, sin), history_rotary=(hc, hs),
                                 q_matrix=qm, kv_matrix=km, out_matrix=om, history_kv_matrix=hm,
                                 **kw)
    keys = torch.cat([k[:, :prefix], hk, k[:, prefix:]], 1)
    vals = torch.cat([v[:, :prefix], hv, v[:, prefix:]], 1)
    kc = torch.cat([cos[:prefix], hc, cos[prefix:]])
    kcs = torch.cat([sin[:prefix], hs, sin[prefix:]])
    kmm = torch.cat([km[:, :prefix], hm, km[:, prefix:]], 1)
    segs = sr.memory_kv_segments(history_rows=2 * C, chunk_rows=C, **kw)
    for qs, qe, ivs in segs:
        idx = torch.cat([torch.arange(a, b) for a, b in ivs])
        qt = h3.rope_prope(q[:, qs:qe], cos[qs:qe], sin[qs:qe], qm[:, qs:qe])
        kt = h3.rope_prope(keys[:, idx], kc[idx], kcs[idx], kmm[:, idx])
        vt = h3.prope_project(vals[:, idx], kmm[:, idx])
        o = h3.prope_project(sr.attention(qt, kt, vt).to(BF), om[:, qs:qe])
        assert torch.equal(got[:, qs:qe], o), (qs, qe)
