"""GPU parity of the H3 transforms (skv_h3_rope_prope) and of the H3 rollout window with them,
against oracle/h3_ref.py (pinned in tests/test_oracle_h3.py).

The transform kernel is bit-exact against the oracle's bf16 chain (rotary on [0, 96), camera
projection on [96, 128)) for every table / matrix dtype, strided BHSD views, broadcast matrices,
row counts that leave a partial block, and in place.  The rollout window (raw chunk-list cache,
window transformed once per chunk, chunk rows per evaluation) follows the oracle's evaluation of
sgf_attention.py:580-659, and the memory-KV layout with per-row transforms (one segmented
launch) the oracle's memory_kv_attention.py:39-140, within the attention bars of
tests/helpers.py.
"""

import pytest
import torch

from oracle import h3_ref as ref
from oracle import segments_ref as sr
from solarwm_amd import h3
from solarwm_amd.segments import H3WindowCache

from .helpers import MAX_ABS, MEAN_ABS

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _say(*a):
    print(*a, flush=True)


def _tables(n, g, dtype):
    theta = torch.rand(n, 48, generator=g, dtype=torch.float64) * 20.0
    c, s = torch.cos(theta), torch.sin(theta)
    return torch.cat([c, c], 1).to(dtype), torch.cat([s, s], 1).to(dtype)


def _matrices(b, n, g):
    return (torch.randn(b, n, 4, 4, generator=g) * 0.6)


def _amplification(vt, matrix):
    """Per-element factor [B, S, H, 128] by which the camera maps scale the bf16 attention bar:
    1 on channels [0, 96); on [96, 128), attention channel j errs in proportion to its
    transformed values (max(1, their RMS over the key rows, per stream and head)) and the
    output block maps those errors with its row of absolute entries (y_i = sum_j m_ij x_j)."""
    B, _, H, _ = vt.shape
    r = vt.double().pow(2).mean(dim=1).sqrt().clamp_min(1.0)[..., 96:].reshape(B, H, 8, 4)
    m = matrix.to(torch.bfloat16).double().abs()  # [B|1, S, 4, 4]
    m = m.expand(B, *m.shape[1:])
    a = torch.einsum("bsij,bhgj->bshgi", m, r).reshape(B, m.shape[1], H, 32)
    return torch.cat([torch.ones(B, m.shape[1], H, 96, dtype=torch.float64), a], dim=-1)


def _bf16_step(x):
    """The spacing of bf16 values at |x| (8 significant bits): 2^(floor(log2 |x|) - 7)."""
    e = torch.frexp(x.double().abs().clamp_min(2.0 ** -126)).exponent
    return torch.ldexp(torch.ones_like(x, dtype=torch.float64), e - 8)


def _assert_propagated_close(got, want, amp):
    """The bf16 attention bars of tests/helpers.py carried through the camera maps: each
    element's error within MAX_ABS times its amplification plus two bf16 steps of the
    output (the attention output and the projected output are each rounded to bf16, here
    and in the reference, and a camera block can double an output's size), the mean within
    MEAN_ABS times the mean amplification."""
    got = got.detach().cpu().double()
    assert torch.isfinite(got).all(), "non-finite attention output"
    want = want.double()
    err = (got - want).abs()
    bar = MAX_ABS * amp + 2 * _bf16_step(want)
    worst = float((err / bar).max())
    _say(f"  max error / bar {worst:.2f}, mean {float(err.mean()):.2e} "
         f"(amplification up to {float(amp.max()):.1f})")
    assert worst <= 1.0, f"max error {worst:.2f} x its bar"
    assert float(err.mean()) <= MEAN_ABS * float(amp.mean()), float(err.mean())


@pytest.mark.parametrize("tdt,mdt,mb,rope,cam", [
    (BF, BF, 2, True, True), (torch.float32, torch.float32, 1, True, True),
    (BF, torch.float32, 2, True, False), (torch.float32, BF, 1, False, True),
    (BF, BF, 2, False, False)])
def test_rope_prope_bit_exact(gpu, tdt, mdt, mb, rope, cam):
    _say("h3 rope_prope", tdt, mdt, mb, rope, cam)
    g = torch.Generator().manual_seed(11)
    B, S, H = 2, 517, 3
    x = torch.randn(B, S, H, 128, generator=g).to(BF)
    cos, sin = _tables(S, g, tdt) if rope else (None, None)
    m = _matrices(mb, S, g).to(mdt) if cam else None
    want = ref.rope_prope(x, cos, sin, m)
    dev = lambda t: None if t is None else t.to(gpu)  # noqa: E731
    got = h3.rope_prope(x.to(gpu), dev(cos), dev(sin), dev(m))
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)
    # strided input: BSHD view of BHSD memory, output into a BHSD-strided view; then in place
    xb = x.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    ob = torch.empty(B, H, S, 128, dtype=BF, device=gpu).transpose(1, 2)
    h3.rope_prope(xb, dev(cos), dev(sin), dev(m), out=ob)
    xi = x.to(gpu)
    h3.rope_prope(xi, dev(cos), dev(sin), dev(m), out=xi)
    torch.cuda.synchronize()
    assert torch.equal(ob.cpu(), want) and torch.equal(xi.cpu(), want)


def test_prope_project_and_qkv_separate(gpu):
    """prope_project on a BHSD view; prope_qkv_separate's matrices from the cameras (the
    reference's bf16 tensor operations, on the GPU) match the oracle's CPU evaluation within a
    bf16 unit, and its projections are bit-exact given those matrices."""
    _say("h3 prope_qkv_separate")
    g = torch.Generator().manual_seed(12)
    B, H, S = 1, 2, 300
    q, k, v = (torch.randn(B, H, S, 128, generator=g).to(BF) for _ in range(3))
    vm = torch.eye(4).repeat(B, S, 1, 1)
    ang = torch.rand(S, generator=g) * 3.0
    vm[0, :, 0, 0], vm[0, :, 0, 2] = torch.cos(ang), torch.sin(ang)
    vm[0, :, 2, 0], vm[0, :, 2, 2] = -torch.sin(ang), torch.cos(ang)
    vm[0, :, :3, 3] = torch.randn(S, 3, generator=g) * 2.0
    ks = torch.eye(3).repeat(B, S, 1, 1)
    qm_o, km_o, om_o = ref.prope_qkv_separate_matrices(vm, ks, vm, ks, BF)
    qm, km, om = h3.prope_qkv_matrices(vm.to(gpu), ks.to(gpu), vm.to(gpu), ks.to(gpu), BF)
    for got, want in ((qm, qm_o), (km, km_o), (om, om_o)):
        torch.testing.assert_close(got.cpu().float(), want.float(), rtol=2 ** -7, atol=2 ** -7)
    qo, ko, vo, out_fn = h3.prope_qkv_separate(q.to(gpu), k.to(gpu), v.to(gpu), query_viewmats=vm.to(gpu),
                                               query_K=ks.to(gpu), key_viewmats=vm.to(gpu),
                                               key_K=ks.to(gpu))
    back = out_fn(vo)
    torch.cuda.synchronize()
    qmc, kmc, omc = qm.cpu(), km.cpu(), om.cpu()
    tr = lambda t: t.transpose(1, 2)  # noqa: E731
    assert torch.equal(tr(qo.cpu()), ref.prope_project(tr(q), qmc))
    assert torch.equal(tr(ko.cpu()), ref.prope_project(tr(k), kmc))
    assert torch.equal(tr(vo.cpu()), ref.prope_project(tr(v), kmc))
    assert torch.equal(tr(back.cpu()), ref.prope_project(ref.prope_project(tr(v), kmc), omc))
    # one camera per row on both sides: the output map undoes the value map (bf16 rounding)
    torch.testing.assert_close(back.cpu().float(), v.float(), rtol=0.05, atol=0.05)


# (37, 2): outputs up to 3.4 after the camera blocks, one of them 2 bf16 units off
@pytest.mark.parametrize("P,nb", [(150, 1), (0, 2), (37, 2)])
def test_h3_window_rollout_vs_oracle(gpu, P, nb):
    """Eight chunks through H3WindowCache (two evaluations each, the second commits) against
    the oracle's transformed window evaluation; history past five chunks rolls off."""
    _say("h3 window rollout", P, nb)
    T, H, cf = 64, 2, 2
    C = cf * T
    g = torch.Generator().manual_seed(13 + P)
    cache = H3WindowCache(num_layers=2, batch=nb, heads=H, frame_tokens=T, prefix_rows=P,
                          chunk_frames=cf, window=5, device=gpu)
    oc = sr.H3RawKVCache()
    pk, pv = (torch.randn(nb, P, H, 128, generator=g).to(BF) for _ in range(2))
    for c in range(8):
        nh = min(c, 5)
        total = P + (nh + 1) * C
        kc, ks = _tables(total, g, BF)
        qc, qs = kc[total - C:].clone(), ks[total - C:].clone()
        kvm = _matrices(nb, total, g)
        qm = _matrices(1, C, g)
        om = _matrices(nb, C, g)
        for commit in (False, True):
            q, k, v = (torch.randn(nb, C, H, 128, generator=g).to(BF) for _ in range(3))
            got = cache.attend(q.to(gpu), k.to(gpu), v.to(gpu), 1, c, prefix=(pk.to(gpu), pv.to(gpu)),
                               q_rotary=(qc.to(gpu), qs.to(gpu)), k_rotary=(kc.to(gpu), ks.to(gpu)),
                               q_matrix=qm.to(gpu), kv_matrix=kvm.to(gpu), out_matrix=om.to(gpu),
                               commit=commit)
            hist = oc.history(1, c)
            keys = torch.cat([pk, *(e[1] for e in hist), k], 1)
            vals = torch.cat([pv, *(e[2] for e in hist), v], 1)
            amp = _amplification(ref.prope_project(vals, kvm), om)
            want = ref.windowed_rollout_attention(q, k, v, pk, pv, oc, 1, c, q_rotary=(qc, qs),
                                                  k_rotary=(kc, ks), q_matrix=qm, kv_matrix=kvm,
                                                  out_matrix=om, commit=commit)
            torch.cuda.synchronize()
            _assert_propagated_close(got, want, amp)
    assert [e[0] for e in cache.history(1, 8)] == [3, 4, 5, 6, 7]
    with pytest.raises(RuntimeError):
        cache.history(0, 2)


@pytest.mark.parametrize("n_bank,audio_rows", [(2, 70), (0, 0)])
def test_h3_memory_kv_vs_oracle(gpu, n_bank, audio_rows):
    """H3WindowCache.attend_memory over three chunks (history rolling in) against the oracle's
    memory-KV evaluation with the same per-row tables and matrices."""
    _say("h3 memory kv", n_bank, audio_rows)
    T, H, cf, text = 64, 2, 2, 100
    C = cf * T
    prefix = text + T + n_bank * T + audio_rows
    g = torch.Generator().manual_seed(21 + n_bank)
    cache = H3WindowCache(num_layers=1, batch=1, heads=H, frame_tokens=T, prefix_rows=prefix,
                          chunk_frames=cf, window=5, device=gpu)
    oc = sr.H3RawKVCache()
    for c in range(3):
        L = prefix + C
        cos, sin = _tables(L, g, BF)
        hrows = min(c, 5) * C
        hc, hs = _tables(hrows, g, BF)
        qm, km, om = (_matrices(1, L, g) for _ in range(3))
        hm = _matrices(1, hrows, g)
        q, k, v = (torch.randn(1, L, H, 128, generator=g).to(BF) for _ in range(3))
        dev = lambda t: t.to(gpu)  # noqa: E731
        got = cache.attend_memory(dev(q), dev(k), dev(v), 0, c, text_rows=text, n_bank=n_bank,
                                  audio_rows=audio_rows, rotary=(dev(cos), dev(sin)),
                                  history_rotary=(dev(hc), dev(hs)) if hrows else None,
                                  q_matrix=dev(qm), kv_matrix=dev(km), out_matrix=dev(om),
                                  history_kv_matrix=dev(hm) if hrows else None, commit=True)
        hist = oc.history(0, c)
        hk = torch.cat([e[1] for e in hist], 1) if hist else k[:, :0]
        hv = torch.cat([e[2] for e in hist], 1) if hist else v[:, :0]
        want = ref.memory_kv_attention(q, k, v, hk, hv, text_rows=text, frame_rows=T,
                                       n_bank=n_bank, audio_rows=audio_rows, rotary=(cos, sin),
                                       history_rotary=(hc, hs), q_matrix=qm, kv_matrix=km,
                                       out_matrix=om, history_kv_matrix=hm)
        hvt = ref.prope_project(hv, hm) if hrows else hv
        amp = _amplification(torch.cat([ref.prope_project(v, km), hvt], 1), om)
        oc.commit(0, c, k[:, prefix:], v[:, prefix:])
        torch.cuda.synchronize()
        _assert_propagated_close(got, want, amp)
