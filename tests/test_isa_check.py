"""The MFMA result-hazard check that gates the library build (solarwm_amd/isa_check.py).

Each case is a small gfx950 listing in hipcc's -S layout.  The first restates the path that once
let a split attention segment read its last row sum too early: the row-sum product, a branch
around the mask block straight to the block that compares the sum, one s_nop 0 in between.
"""

from solarwm_amd import isa_check

HEAD = "_ZN3skv4testEv:                        ; @_ZN3skv4testEv\n"
TAIL = "\ts_endpgm\n.Lfunc_end0:\n"


def _check(body: str):
    return isa_check.check_listing(HEAD + body + TAIL)


ROWSUM_BRANCH = """\
\tv_mfma_f32_16x16x128_f8f6f4 v[28:31], v[180:187], v[20:27], 0
\ts_cbranch_vccnz .LBB0_2
; %bb.1:
\ts_lshl_b32 s2, s29, 6
\ts_mul_i32 s3, s23, s68
\ts_add_i32 s3, s3, s2
\ts_add_i32 s8, s2, 64
\ts_cmp_gt_i32 s8, s31
\ts_cselect_b64 s[8:9], -1, 0
\ts_add_i32 s10, s3, 64
\ts_cmp_gt_i32 s10, s96
\ts_cselect_b64 s[10:11], -1, 0
\ts_or_b64 s[8:9], s[8:9], s[10:11]
\ts_andn2_b64 vcc, exec, s[8:9]
\tv_cndmask_b32 v66, v254, v66, vcc
.LBB0_2:
{wait}\tv_cmp_nge_f32_e32 vcc, s97, v28
"""


def test_branch_around_a_block_is_a_short_path():
    bad = _check(ROWSUM_BRANCH.format(wait="\ts_nop 0\n"))
    (paths,) = bad.values()
    assert len(paths) == 1
    p = paths[0]
    assert p.waited == 2 and p.needed == 12 and "v_cmp_nge_f32" in p.reader


def test_spelled_out_wait_clears_it():
    # s_nop 7 + s_nop 4 = 13 wait states, plus the branch
    assert _check(ROWSUM_BRANCH.format(wait="\ts_nop 7\n\ts_nop 4\n")) == {}


def test_fall_through_path_alone_is_long_enough():
    # without the branch the 12 SALU ops and the select in between cover the 8-pass product
    body = ROWSUM_BRANCH.format(wait="").replace("\ts_cbranch_vccnz .LBB0_2\n", "")
    assert _check(body) == {}


def test_sixteen_pass_product_needs_twenty():
    body = ("\tv_mfma_f32_32x32x64_f8f6f4 v[34:49], v[2:9], v[146:153], 0\n"
            "\ts_nop 7\n\ts_nop 7\n\ts_nop 2\n"        # 19 wait states
            "\tv_cndmask_b32 v34, v28, v34, vcc\n")
    (paths,) = _check(body).values()
    assert paths[0].waited == 19 and paths[0].needed == 20
    assert _check(body.replace("s_nop 2", "s_nop 3")) == {}


def test_a_later_product_counts_its_passes():
    body = ("\tv_mfma_f32_32x32x64_f8f6f4 v[34:49], v[2:9], v[146:153], 0\n"
            "\tv_mfma_f32_32x32x64_f8f6f4 v[50:65], v[2:9], v[154:161], 0\n"
            "\ts_nop 3\n"
            "\tv_cndmask_b32 v34, v28, v34, vcc\n")
    assert _check(body) == {}


def test_accumulator_chain_is_left_to_the_hardware():
    body = ("\tv_mfma_f32_32x32x64_f8f6f4 v[34:49], v[2:9], v[146:153], 0\n"
            "\tv_mfma_f32_32x32x64_f8f6f4 v[34:49], v[10:17], v[154:161], v[34:49]\n"
            + "\ts_nop 7\n" * 3 +
            "\tv_mov_b32_e32 v3, v34\n")
    assert _check(body) == {}


def test_load_that_overwrites_the_result_needs_one_less():
    body = ("\tv_mfma_f32_32x32x16_f16 v[98:113], v[182:185], v[162:165], v[98:113]\n"
            "\ts_nop 7\n\ts_nop 2\n"                   # 11 wait states
            "\tds_read_b128 v[98:101], v97\n")
    assert _check(body) == {}
    (paths,) = _check(body.replace("ds_read_b128 v[98:101], v97",
                                   "v_mov_b32_e32 v98, 0")).values()
    assert paths[0].waited == 11 and paths[0].needed == 12


def test_loop_back_edge_is_followed():
    body = (".LBB0_1:\n"
            "\tv_add_f32_e32 v1, v28, v2\n"
            "\ts_add_i32 s0, s0, 1\n"
            "\tv_mfma_f32_16x16x128_f8f6f4 v[28:31], v[180:187], v[20:27], 0\n"
            "\ts_cmp_lt_i32 s0, s1\n"
            "\ts_cbranch_scc1 .LBB0_1\n")
    (paths,) = _check(body).values()
    assert "v_add_f32" in paths[0].reader and paths[0].waited == 2


def test_unknown_product_form_is_reported():
    body = "\tv_mfma_f32_4x4x4_16b_f16 v[0:3], v[4:5], v[6:7], 0\n"
    (paths,) = _check(body).values()
    assert "unknown" in paths[0].reader


def test_real_listing_from_hipcc(tmp_path):
    """The walk on hipcc's own -S output: a row-sum-shaped product whose result a VALU op reads
    behind a branch.  hipcc's listing passes; with its s_nop lines deleted the read is short."""
    import re
    import shutil
    import subprocess

    import pytest

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not shutil.os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    src = tmp_path / "k.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "typedef int i32x8 __attribute__((ext_vector_type(8)));\n"
        "typedef float f32x4 __attribute__((ext_vector_type(4)));\n"
        'extern "C" __global__ void rowsum_branch(const int* p, float* out, int n) {\n'
        "  i32x8 a, b;\n"
        "  for (int i = 0; i < 8; ++i) { a[i] = p[threadIdx.x * 8 + i]; b[i] = p[512 + threadIdx.x * 8 + i]; }\n"
        "  f32x4 c = {0.f, 0.f, 0.f, 0.f};\n"
        "  f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);\n"
        "  float x = 0.f;\n"
        "  if (n > 3) x = out[threadIdx.x] * 2.f;\n"
        "  out[threadIdx.x] = d[0] + x;\n"
        "}\n")
    asm = tmp_path / "k.s"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "--cuda-device-only", "-S", str(src),
                    "-o", str(asm)], check=True, capture_output=True)
    listing = asm.read_text()
    assert [name for name, _ in isa_check.functions(listing)] == ["rowsum_branch"]
    assert isa_check.check_listing(listing) == {}
    stripped = re.sub(r"\n\ts_nop \d+", "", listing)
    (paths,) = isa_check.check_listing(stripped).values()
    assert any(p.needed == 12 and p.waited < 12 for p in paths), [str(p) for p in paths]


def test_pass_table_matches_hipcc(tmp_path):
    """The wait each MFMA form needs (its passes + EXTRA_WAIT) is exactly what hipcc's hazard pass
    puts between the product and a VALU read of its result in straight-line code."""
    import shutil
    import subprocess

    import pytest

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not shutil.os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    head = ("#include <hip/hip_runtime.h>\n"
            "typedef int i32x8 __attribute__((ext_vector_type(8)));\n"
            "typedef float f32x4 __attribute__((ext_vector_type(4)));\n"
            "typedef float f32x16 __attribute__((ext_vector_type(16)));\n"
            "typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));\n"
            "typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));\n")
    forms = {  # kernel name: (operand type, accumulator type, product)
        "k_f8_32": ("i32x8", "f32x16", "__builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0)"),
        "k_f8_16": ("i32x8", "f32x4", "__builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0)"),
        "k_bf16_32": ("bf16x8", "f32x16", "__builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0)"),
        "k_f16_32": ("f16x8", "f32x16", "__builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0)"),
        "k_bf16_16": ("bf16x8", "f32x4", "__builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0)"),
    }
    body = head + "".join(
        f'extern "C" __global__ void {name}(const {op}* p, float* out) {{\n'
        f"  {op} a = p[threadIdx.x], b = p[64 + threadIdx.x];\n"
        f"  {acc} c = {{}};\n  {acc} d = {call};\n  out[threadIdx.x] = d[0] + 1.0f;\n}}\n"
        for name, (op, acc, call) in forms.items())
    src = tmp_path / "k.hip"
    src.write_text(body)
    asm = tmp_path / "k.s"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "--cuda-device-only", "-S", str(src),
                    "-o", str(asm)], check=True, capture_output=True)
    seen = {}
    for name, lines in isa_check.functions(asm.read_text()):
        ins = [t for t in (ln.split(";")[0].strip() for ln in lines) if t and not t.startswith(".")
               and not t.endswith(":")]
        i = next(k for k, t in enumerate(ins) if "mfma" in t.split()[0])
        op = ins[i].split()[0]
        waited = 0
        for t in ins[i + 1:]:
            if t.startswith("v_add_f32"):
                break
            waited += int(t.split()[1]) + 1 if t.startswith("s_nop") else 1
        seen[op] = waited
        assert waited == isa_check.PASSES[op] + isa_check.EXTRA_WAIT, (name, op, waited)
    assert len(seen) == len(forms)
