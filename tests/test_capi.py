"""libsolarkv.so loads, exports every entry point include/solarkv.h declares, and rejects bad
arguments with the documented status codes before touching a GPU."""

import ctypes
import re
from pathlib import Path

import pytest

from solarwm_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "solarkv.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(skv_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_entry_points():
    assert _declared() == sorted(_lib.SIGNATURES)


def test_library_exports_every_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.skv_version() >= 100


def test_constants_match_header():
    text = HEADER.read_text()
    for name in ("SKV_MAX_APPEND_FRAMES", "SKV_MAX_FRAMES"):
        m = re.search(rf"#define {name} (\d+)", text)
        assert int(m.group(1)) == getattr(_lib, name)
    for name in ("SKV_F32", "SKV_BF16", "SKV_FP8_E4M3", "SKV_MASK_NONE", "SKV_MASK_CHUNK_CAUSAL",
                 "SKV_OK", "SKV_E_ARG", "SKV_E_UNSUPPORTED", "SKV_E_LAUNCH"):
        m = re.search(rf"\b{name} = (-?\d+)", text)
        assert int(m.group(1)) == getattr(_lib, name), name


def _slots(*v):
    return _lib.int32_array(v)


def test_argument_errors_do_not_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation
    st = lib.skv_append(None, fake, _lib.SKV_BF16, 0, 0, 0, 0, fake, fake, None, None,
                        _lib.SKV_BF16, 4, _slots(0), 1, 1, 1, 128, 64, None)
    assert st == _lib.SKV_E_ARG and b"null" in lib.skv_last_error()
    st = lib.skv_append(fake, fake, _lib.SKV_BF16, 0, 0, 0, 0, fake, fake, None, None,
                        _lib.SKV_BF16, 4, _slots(0), 1, 1, 1, 64, 64, None)
    assert st == _lib.SKV_E_UNSUPPORTED and b"head_dim" in lib.skv_last_error()
    st = lib.skv_append(fake, fake, _lib.SKV_BF16, 8, 8, 8, 0, fake, fake, None, None,
                        _lib.SKV_BF16, 4, _slots(7), 1, 1, 1, 128, 64, None)
    assert st == _lib.SKV_E_ARG and b"dst_slots" in lib.skv_last_error()
    st = lib.skv_append(fake, fake, _lib.SKV_BF16, 8, 8, 8, 0, fake, fake, None, None,
                        _lib.SKV_FP8_E4M3, 4, _slots(0), 1, 1, 1, 128, 64, None)
    assert st == _lib.SKV_E_ARG and b"scale" in lib.skv_last_error()
    st = lib.skv_gather(fake, fake, _lib.SKV_BF16, 4, _slots(0), 1, 1, 1, 128, 64, fake, fake,
                        3, 8, 8, None)
    assert st == _lib.SKV_E_ARG and b"multiples of 8" in lib.skv_last_error()
    st = lib.skv_attention(fake, _lib.SKV_BF16, 8, 8, 8, fake, fake, None, None, _lib.SKV_BF16,
                           4, _slots(0), 0, 1, 1, 128, 16, 64, 0.1, 0, 0, 0, fake, 8, 8, 8, None)
    assert st == _lib.SKV_E_ARG and b"empty key window" in lib.skv_last_error()
    st = lib.skv_attention(fake, _lib.SKV_BF16, 8, 8, 8, fake, fake, None, None, _lib.SKV_BF16,
                           4, _slots(0), 1, 1, 1, 128, 16, 64, 0.1, 5, 0, 0, fake, 8, 8, 8, None)
    assert st == _lib.SKV_E_ARG and b"mask_mode" in lib.skv_last_error()
    st = lib.skv_attention(fake, _lib.SKV_BF16, 8, 8, 8, fake, fake, None, None, _lib.SKV_BF16,
                           4, _slots(9), 1, 1, 1, 128, 16, 64, 0.1, 0, 0, 0, fake, 8, 8, 8, None)
    assert st == _lib.SKV_E_ARG and b"frame_slots" in lib.skv_last_error()


def test_python_wrapper_raises_valueerror():
    with pytest.raises(ValueError):
        _lib.check("skv_append", _lib.SKV_E_ARG)
    with pytest.raises(_lib.SolarKVError):
        _lib.check("skv_append", _lib.SKV_E_LAUNCH)


def test_signature_arity_matches_header():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, (_, argtypes) in _lib.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\(([^)]*)\)\s*;", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(argtypes), name


def test_rope_argument_errors_do_not_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    # fp8 pools: the flat entry point carries no copy scales (skv_append_ex does)
    st = lib.skv_append_rope(fake, fake, _lib.SKV_BF16, 8, 8, 8, 0, fake, fake, _lib.SKV_FP8_E4M3,
                             4, _slots(0), 1, 1, 1, 128, 64, fake, fake, 8, 8, None)
    assert st == _lib.SKV_E_ARG and b"kr_scale" in lib.skv_last_error()
    # the spatial grid must tile the frame
    st = lib.skv_append_rope(fake, fake, _lib.SKV_BF16, 8, 8, 8, 0, fake, fake, _lib.SKV_BF16,
                             4, _slots(0), 1, 1, 1, 128, 64, fake, fake, 8, 7, None)
    assert st == _lib.SKV_E_ARG and b"grid" in lib.skv_last_error()
    st = lib.skv_append_rope(fake, fake, _lib.SKV_BF16, 8, 8, 8, 0, fake, fake, _lib.SKV_BF16,
                             4, _slots(0), 1, 1, 1, 128, 64, None, fake, 8, 8, None)
    assert st == _lib.SKV_E_ARG and b"kr_pool" in lib.skv_last_error()
    args = dict(q_len=128, T=64, pool=_lib.SKV_BF16, nq=2, rope_t=fake)

    def attn(**kw):
        a = dict(args, **kw)
        return lib.skv_attention_rope(fake, _lib.SKV_BF16, 8, 8, 8, fake, fake, a["pool"], 4,
                                      _slots(0), 1, 1, 1, 128, a["q_len"], a["T"], 0.1, 0, 0, 0,
                                      fake, 8, 8, 8, fake, 8, 8, a["rope_t"], a["nq"], None)
    assert attn(pool=_lib.SKV_F32) == _lib.SKV_E_UNSUPPORTED and b"bf16" in lib.skv_last_error()
    assert attn(nq=3) == _lib.SKV_E_ARG and b"n_qframes" in lib.skv_last_error()
    assert attn(rope_t=None) == _lib.SKV_E_ARG and b"rope_t" in lib.skv_last_error()


def test_prope_argument_errors_do_not_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)

    def app(**kw):
        a = dict(pool=_lib.SKV_BF16, kx=fake, vx=fake, xf=fake, gw=8)
        a.update(kw)
        return lib.skv_append_prope(fake, fake, _lib.SKV_BF16, 8, 8, 8, 0, fake, fake, a["pool"], 4,
                                    _slots(0), 1, 1, 1, 128, 64, a["kx"], a["vx"], fake, 8,
                                    a["gw"], a["xf"], None)
    assert app(vx=None) == _lib.SKV_E_ARG and b"vx_pool" in lib.skv_last_error()
    assert app(xf=None) == _lib.SKV_E_ARG and b"kv_xform" in lib.skv_last_error()
    assert app(pool=_lib.SKV_F32) == _lib.SKV_E_UNSUPPORTED
    assert app(gw=7) == _lib.SKV_E_ARG and b"grid" in lib.skv_last_error()

    def attn(**kw):
        a = dict(q_len=128, T=64, pool=_lib.SKV_BF16, nq=2, xt=fake, xs=fake, xo=fake, gh=8, gw=8)
        a.update(kw)
        return lib.skv_attention_prope(fake, _lib.SKV_BF16, 8, 8, 8, fake, fake, a["pool"], 4,
                                       _slots(0), 1, 1, 1, 128, a["q_len"], a["T"], 0.1, 0, 0, 0,
                                       fake, 8, 8, 8, fake, a["gh"], a["gw"], a["xt"], a["xs"],
                                       a["xo"], a["nq"], None)
    assert attn(xt=None) == _lib.SKV_E_ARG and b"q_xform_t" in lib.skv_last_error()
    assert attn(xo=None) == _lib.SKV_E_ARG and b"out_xform" in lib.skv_last_error()
    assert attn(pool=_lib.SKV_F32) == _lib.SKV_E_UNSUPPORTED
    assert attn(q_len=60, T=30, gh=5, gw=6) == _lib.SKV_E_UNSUPPORTED  # frames under 64 tokens
    assert attn(nq=3) == _lib.SKV_E_ARG and b"n_qframes" in lib.skv_last_error()


@pytest.mark.parametrize("cname,pyname", [("skv_append_desc", "AppendDesc"),
                                          ("skv_attention_desc", "AttentionDesc"),
                                          ("skv_launch_plan", "LaunchPlan"),
                                          ("skv_h3_xform_desc", "H3XformDesc")])
def test_descriptor_layout_matches_header(tmp_path, cname, pyname):
    """The ctypes mirrors of the descriptor structs have the C compiler's size and offsets."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    py = getattr(_lib, pyname)
    fields = [f for f, _ in py._fields_]
    src = tmp_path / "layout.c"
    src.write_text(
        f'#include <stdio.h>\n#include <stddef.h>\n#include "solarkv.h"\nint main(void) {{\n'
        f'  printf("%zu\\n", sizeof({cname}));\n'
        + "".join(f'  printf("%zu\\n", offsetof({cname}, {f}));\n' for f in fields)
        + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True,
                                          text=True).stdout.split()]
    assert got[0] == ctypes.sizeof(py)
    assert got[1:] == [getattr(py, f).offset for f in fields]


def test_extended_entry_points_reject_bad_options():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    assert lib.skv_append_ex(None, None) == _lib.SKV_E_ARG
    d = _lib.AppendDesc(k_new=fake, v_new=fake, src_dtype=_lib.SKV_BF16, src_sb=8, src_st=8,
                        src_sh=8, k_pool=fake, v_pool=fake, pool_dtype=_lib.SKV_BF16, n_slots=4,
                        dst_slots=_slots(0), n_frames=1, batch=1, heads=1, head_dim=128,
                        frame_tokens=64, k_inv_rms=fake)
    assert lib.skv_append_ex(ctypes.byref(d), None) == _lib.SKV_E_ARG  # weight missing
    assert b"k_norm_weight" in lib.skv_last_error()
    d.k_norm_weight, d.k_rms_stride_b = fake, 32
    assert lib.skv_append_ex(ctypes.byref(d), None) == _lib.SKV_E_ARG  # stride too short
    d.k_inv_rms = d.k_norm_weight = None
    d.vx_pool = fake
    assert lib.skv_append_ex(ctypes.byref(d), None) == _lib.SKV_E_ARG  # PRoPE without kr_pool
    a = _lib.AttentionDesc(q=fake, q_dtype=_lib.SKV_BF16, q_sb=8, q_st=8, q_sh=8, k_pool=fake,
                           v_pool=fake, pool_dtype=_lib.SKV_BF16, n_slots=4, frame_slots=_slots(0),
                           n_frames=1, batch=1, heads=1, head_dim=128, q_len=64, frame_tokens=64,
                           softmax_scale=0.1, out=fake, out_sb=8, out_st=8, out_sh=8,
                           q_norm_weight=fake)
    assert lib.skv_attention_ex(ctypes.byref(a), None) == _lib.SKV_E_ARG  # q_inv_rms missing
    a.q_inv_rms, a.q_rms_stride_b = fake, 32
    assert lib.skv_attention_ex(ctypes.byref(a), None) == _lib.SKV_E_ARG  # stride < q_len
    a.q_rms_stride_b, a.rope_t, a.q_xform_t = 64, fake, fake
    assert lib.skv_attention_ex(ctypes.byref(a), None) == _lib.SKV_E_ARG  # both RoPE modes
    st = lib.skv_rms_rows(fake, _lib.SKV_BF16, 8, 8, 8, 1, 4, 1, 64, 1e-6, fake, None)
    assert st == _lib.SKV_E_UNSUPPORTED
    st = lib.skv_rms_rows(fake, _lib.SKV_BF16, 8, 8, 8, 1, 4, 1, 128, -1.0, fake, None)
    assert st == _lib.SKV_E_ARG


def _attn_desc(B, H, Lq, T, nf, pool=_lib.SKV_BF16, mask=_lib.SKV_MASK_NONE):
    fake = ctypes.c_void_p(0x1000)
    slots = _slots(*range(nf))
    d = _lib.AttentionDesc(q=fake, q_dtype=_lib.SKV_BF16, q_sb=8, q_st=8, q_sh=8, k_pool=fake,
                           v_pool=fake, pool_dtype=pool, n_slots=nf + 3, frame_slots=slots,
                           n_frames=nf, batch=B, heads=H, head_dim=128, q_len=Lq, frame_tokens=T,
                           softmax_scale=0.1, mask_mode=mask, chunk_tokens=Lq, out=fake, out_sb=8,
                           out_st=8, out_sh=8)
    if pool == _lib.SKV_FP8_E4M3:
        d.k_scale = d.v_scale = fake
    return d, slots


def _plan(d):
    lib = _lib.load()
    plan = _lib.LaunchPlan()
    assert lib.skv_attention_plan(ctypes.byref(d), ctypes.byref(plan)) == _lib.SKV_OK
    return plan


SPLIT_BYTES = 2 * 256 * 256 * 130 * 4  # 2 records x 256 rows x (128 O + max + sum) per CU


@pytest.mark.parametrize("name,B,H,Lq,T,nf,pool,want", [
    # the benchmark's launch shapes (256-CU MI355X): (waves per group, split, workgroups)
    ("c2", 1, 12, 4680, 1560, 21, _lib.SKV_BF16, (8, 0, 228)),
    ("c3", 1, 24, 2640, 880, 21, _lib.SKV_BF16, (8, 1, 256)),
    ("c4", 1, 40, 4680, 1560, 29, _lib.SKV_BF16, (8, 0, 760)),
    ("c5", 4, 12, 4680, 1560, 21, _lib.SKV_FP8_E4M3, (8, 2, 1024)),
    ("one_frame", 1, 12, 1560, 1560, 21, _lib.SKV_BF16, (8, 1, 256)),
    ("one_frame_fp8", 4, 12, 1560, 1560, 21, _lib.SKV_FP8_E4M3, (8, 1, 256)),
])
def test_launch_plans_of_benchmark_shapes(name, B, H, Lq, T, nf, pool, want):
    """skv_attention_plan reports the launcher's choice without launching (the device count
    falls back to MI355X's 256 CUs when no GPU is visible); the split is taken only with a
    workspace of the reported size."""
    lib = _lib.load()
    d, _keep = _attn_desc(B, H, Lq, T, nf, pool)
    bare = _plan(d)
    assert bare.split == 0 and bare.workspace_bytes == (SPLIT_BYTES if want[1] else 0)
    if want[1]:
        d.workspace, d.workspace_bytes = 0x2000, bare.workspace_bytes
    plan = _plan(d)
    assert (plan.waves_per_group, plan.split, plan.n_workgroups) == want, name
    if want[1]:
        d.workspace_bytes = bare.workspace_bytes - 4
        assert lib.skv_attention_plan(ctypes.byref(d), ctypes.byref(_lib.LaunchPlan())) == _lib.SKV_E_ARG
        assert b"smaller" in lib.skv_last_error()
        d.workspace, d.workspace_bytes = 0x2008, bare.workspace_bytes
        assert lib.skv_attention_plan(ctypes.byref(d), ctypes.byref(_lib.LaunchPlan())) == _lib.SKV_E_ARG
        assert b"aligned" in lib.skv_last_error()


@pytest.mark.parametrize("name,B,H,Lq,T,nf,pool,want", [
    # 64-key tiles per query tile: packed across frame boundaries for whole bf16 / f16 frames of
    # T = 8k tokens (T not a multiple of 64), frame-aligned otherwise
    ("c2", 1, 12, 4680, 1560, 21, _lib.SKV_BF16, 512),        # 32760 keys, not 21 x 25 = 525
    ("c3", 1, 24, 2640, 880, 21, _lib.SKV_BF16, 289),         # 18480 keys, not 21 x 14 = 294
    ("f16", 1, 2, 300, 72, 7, _lib.SKV_F16, 8),               # 504 keys, not 7 x 2 = 14
    ("c5_fp8", 4, 12, 4680, 1560, 21, _lib.SKV_FP8_E4M3, 525),  # per-frame scales: aligned
    ("f32", 1, 2, 390, 1560, 3, _lib.SKV_F32, 75),            # register staging: aligned
    ("t100", 1, 2, 300, 100, 5, _lib.SKV_BF16, 10),           # T % 8 != 0: aligned
    ("t128", 1, 2, 300, 128, 5, _lib.SKV_BF16, 10),           # no padding to remove
])
def test_plans_report_packed_key_tiles(name, B, H, Lq, T, nf, pool, want):
    d, _keep = _attn_desc(B, H, Lq, T, nf, pool)
    if pool == _lib.SKV_F16:
        d.q_dtype = _lib.SKV_F16  # f16 pools multiply f16 (or f32) queries
    assert _plan(d).key_tiles == want, name


def test_packing_needs_a_pool_under_4gb_and_whole_frames():
    # H40 x 1600 rows x 256 B = 16.4 MB per slot: 263 slots make a pool over 4 GB, 262 do not
    d, _keep = _attn_desc(1, 40, 4680, 1560, 3)
    assert _plan(d).key_tiles == 74  # ceil(3 x 1560 / 64)
    d.n_slots = 263
    assert _plan(d).key_tiles == 75
    d.n_slots = 262
    assert _plan(d).key_tiles == 74
    lens = _slots(1560, 1000, 1560)  # a ragged frame keeps frame-aligned tiles
    d.frame_lens = lens
    assert _plan(d).key_tiles == 75


def test_masked_launches_never_split():
    d, _keep = _attn_desc(1, 12, 1560, 1560, 21, mask=_lib.SKV_MASK_CHUNK_CAUSAL)
    d.workspace, d.workspace_bytes = 0x2000, SPLIT_BYTES
    plan = _plan(d)
    assert plan.split == 0 and plan.workspace_bytes == 0


def test_append_workspace_query():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    slots = _slots(0, 1, 2)

    def need(B, H, T, pool):
        d = _lib.AppendDesc(k_new=fake, v_new=fake, src_dtype=_lib.SKV_BF16, src_sb=8, src_st=8,
                            src_sh=8, k_pool=fake, v_pool=fake, k_scale=fake, v_scale=fake,
                            pool_dtype=pool, n_slots=8, dst_slots=slots, n_frames=3, batch=B,
                            heads=H, head_dim=128, frame_tokens=T)
        out = ctypes.c_int64(-1)
        assert lib.skv_append_workspace_size(ctypes.byref(d), ctypes.byref(out)) == _lib.SKV_OK
        return out.value

    # C5: 3 frames x 4 streams x 12 heads x (K, V) = 288 units: the larger of the one-pass
    # kernel's cells (a 128 B header + up to 512 B per unit) and the tile grids' maxima (one
    # float per 64-token tile, 25 per unit)
    assert need(4, 12, 1560, _lib.SKV_FP8_E4M3) == max(128 + 288 * 512, 288 * 25 * 4)
    assert need(1, 2, 8000, _lib.SKV_FP8_E4M3) == max(128 + 12 * 512, 12 * 125 * 4)
    assert need(4, 12, 1560, _lib.SKV_BF16) == 0
    assert need(16, 24, 1560, _lib.SKV_FP8_E4M3) == 0  # 2304 units fill the chip per unit
    assert lib.skv_append_workspace_size(None, None) == _lib.SKV_E_ARG


def test_fp8_copy_workspace_and_arguments():
    """fp8 pools with RoPE / PRoPE copies: the copies' tile maxima (one float per 64-token tile
    of each copied unit) join the workspace query, the copies need the workspace and their own
    scales, all checked before anything launches."""
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    slots = _slots(0, 1, 2)
    hw = (ctypes.c_float * 8)()

    def desc(B, H, T, gh, prope=False):
        d = _lib.AppendDesc(k_new=fake, v_new=fake, src_dtype=_lib.SKV_BF16, src_sb=8, src_st=8,
                            src_sh=8, k_pool=fake, v_pool=fake, k_scale=fake, v_scale=fake,
                            pool_dtype=_lib.SKV_FP8_E4M3, n_slots=8, dst_slots=slots, n_frames=3,
                            batch=B, heads=H, head_dim=128, frame_tokens=T, kr_pool=fake,
                            rope_hw=ctypes.cast(hw, ctypes.c_void_p), grid_h=gh, grid_w=T // gh,
                            kr_scale=fake)
        if prope:
            d.vx_pool, d.kv_xform, d.vx_scale = fake, fake, fake
        return d

    def need(d):
        out = ctypes.c_int64(-1)
        assert lib.skv_append_workspace_size(ctypes.byref(d), ctypes.byref(out)) == _lib.SKV_OK
        return out.value

    # 2304 raw units fill the chip (no raw workspace); the K copy: 3 x 16 x 24 units x 25 tiles
    assert need(desc(16, 24, 1560, 30)) == 3 * 16 * 24 * 25 * 4
    assert need(desc(16, 24, 1560, 30, prope=True)) == 2 * 3 * 16 * 24 * 25 * 4
    # C5: the raw one-pass cells are larger than the copy maxima
    assert need(desc(4, 12, 1560, 30)) == max(128 + 288 * 512, 144 * 25 * 4)
    d = desc(16, 24, 1560, 30)
    assert lib.skv_append_ex(ctypes.byref(d), None) == _lib.SKV_E_ARG  # no workspace
    assert b"workspace" in lib.skv_last_error()
    d = desc(4, 12, 1560, 30)
    d.kr_scale = None
    assert lib.skv_append_ex(ctypes.byref(d), None) == _lib.SKV_E_ARG
    assert b"kr_scale" in lib.skv_last_error()
    d = desc(4, 12, 1560, 30, prope=True)
    d.vx_scale = None
    assert lib.skv_append_ex(ctypes.byref(d), None) == _lib.SKV_E_ARG
    assert b"vx_scale" in lib.skv_last_error()


def test_segmented_launch_plans_and_arguments():
    """One launch for several query segments: each segment's q-tiles start at its first row (8
    waves, 256 rows), the grid holds every segment's q-tiles, the key split is never taken and
    the reported key tiles are the longest segment's; bad tables are rejected before anything
    launches."""
    from solarwm_amd.segments import teacher_forcing_frame_lists

    lib = _lib.load()
    # the bench's teacher-forcing shape: [clean | noisy] x 6 frames of 1560 tokens, chunks of 3
    lists = teacher_forcing_frame_lists(num_frames=6, num_frame_per_block=3,
                                        max_prior_clean_chunks=1, sink_size=3)
    assert [len(f) for _, f in lists] == [3, 6, 3, 6]
    frames = [f for _, fr in lists for f in fr]
    d, _keep = _attn_desc(1, 12, 4 * 4680, 1560, len(frames))
    table = _slots(*frames)
    rows, nfs = _slots(*[4680] * 4), _slots(*[len(f) for _, f in lists])
    d.frame_slots, d.n_slots = table, 12
    d.seg_rows, d.seg_frames, d.n_segments = rows, nfs, 4
    d.workspace, d.workspace_bytes = 0x2000, SPLIT_BYTES
    plan = _plan(d)
    assert (plan.waves_per_group, plan.split, plan.n_workgroups) == (8, 0, 4 * 19 * 12)
    assert plan.workspace_bytes == 0
    assert plan.key_tiles == -(-6 * 1560 // 64)  # packed tiles of the 6-frame lists
    # ragged segment rows: 300 rows take 2 q-tiles, 1 row takes 1
    d2, _k2 = _attn_desc(2, 3, 301, 64, 3)
    r2, f2 = _slots(300, 1), _slots(2, 1)
    d2.seg_rows, d2.seg_frames, d2.n_segments = r2, f2, 2
    plan = _plan(d2)
    assert (plan.waves_per_group, plan.n_workgroups, plan.key_tiles) == (8, 3 * 3 * 2, 2)

    def err(desc, code, text):
        assert lib.skv_attention_plan(ctypes.byref(desc), ctypes.byref(_lib.LaunchPlan())) == code
        assert text in lib.skv_last_error(), lib.skv_last_error()

    d2.n_segments = _lib.SKV_MAX_SEGMENTS + 1
    err(d2, _lib.SKV_E_ARG, b"n_segments")
    d2.n_segments, d2.seg_frames = 2, None
    err(d2, _lib.SKV_E_ARG, b"seg_frames")
    bad = _slots(299, 1)
    d2.seg_frames, d2.seg_rows = f2, bad
    err(d2, _lib.SKV_E_ARG, b"q_len=301")
    zero = _slots(301, 0)
    d2.seg_rows, d2.seg_frames = r2, zero
    err(d2, _lib.SKV_E_ARG, b"must be >= 1")
    d2.seg_frames = f2
    d2.mask_mode = _lib.SKV_MASK_CHUNK_CAUSAL
    err(d2, _lib.SKV_E_UNSUPPORTED, b"mask NONE")
    d3, _k3 = _attn_desc(1, 2, 301, 64, 3, pool=_lib.SKV_FP8_E4M3)
    d3.seg_rows, d3.seg_frames, d3.n_segments = r2, f2, 2
    err(d3, _lib.SKV_E_UNSUPPORTED, b"bf16 pools")


def test_library_launches_nothing_cooperatively():
    """No entry point launches a kernel cooperatively: the one-pass fp8 append sizes its grid
    from the occupancy query and launches it plainly (its waits are bounded).  A cooperative
    launch of that kernel, in a build that was never part of the library, was running when a
    rocprofv3-traced process crashed in the runtime's exit handlers."""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    res = subprocess.run([nm, "-D", "--undefined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True)
    imports = {w.split("@")[0] for w in res.stdout.split() if w != "U"}
    assert "hipLaunchKernel" in imports or "__hipPushCallConfiguration" in imports
    assert not {s for s in imports if "Cooperative" in s}, imports
