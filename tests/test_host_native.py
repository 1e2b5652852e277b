"""Host side of the drop-in boundary, on the CPU: the C-ABI library loads and
exports every function include/jacq_kivi.h declares, and its host-only
entry points (validators, planner, versions) match the reference's tables.
No GPU call is made here.

Fixtures and tables:
  * tests/golden/gpu_boundary_probe.json -- the reference's own width probe
    (validation/vllm-2026-11-03/gpu-boundary-probe.json:1-62), also the cases
    of tests/test_runtime_guards.py:164-201;
  * byte math of tests/test_layout_and_scaffold.py:162-174;
  * jac_launch argument order of tests/test_launch_signature.py:37-57;
  * plan_batched_write (source_patch.py:504-553): no reference test pins its
    outputs, so it is pinned by its invariants and against the oracle's C
    restatement.
"""
from __future__ import annotations

import ctypes
import json
import os
import re

import numpy as np
import pytest
import torch

from jacq_amd import abi, geometry, kivi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "jacq_kivi.h")


def header_functions() -> dict[str, list[str]]:
    """name -> parameter identifiers of every function the header declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*([a-z_0-9]+)\s*\(([^)]*)\)\s*;",
                         text, flags=re.M):
        params = []
        for p in m.group(2).split(","):
            p = p.strip()
            if p in ("", "void"):
                continue
            params.append(re.findall(r"[A-Za-z_][A-Za-z0-9_]*$", p)[0])
        out[m.group(1)] = params
    return out


@pytest.fixture(scope="module")
def native():
    if not os.path.exists(kivi.library_path()):
        pytest.fail(f"{kivi.library_path()} missing: run `python -m jacq_amd.build`")
    return kivi.lib()


def geo(**kw) -> kivi.Geometry:
    base = dict(num_heads=40, num_kv_heads=8, head_dim=128, page_size=32, group_size=32,
                residual=128, max_pages_per_seq=124, num_pages=1000)
    base.update(kw)
    return kivi.Geometry(*base.values())


def test_header_declares_the_reference_symbols():
    fns = header_functions()
    for name in ("jac_launch", "jac_launch_tp2_local", "jac_launch_batched",
                 "jac_launch_batched_tp2_local", "jac_launch_cache_write",
                 "jac_launch_cache_write_batched", "kivi_cache_write_launch",
                 "kivi_cache_write_batched_launch", "jac_launch_sparse_retained",
                 "jac_launch_sparse_retained_tp2_local"):
        assert name in fns, name
    ext = sorted(n for n in fns if n.startswith("jacq_kivi_"))
    assert ext == sorted([
        "jacq_kivi_abi_version", "jacq_kivi_ext_version", "jacq_kivi_last_error",
        "jacq_kivi_check_geometry", "jacq_kivi_max_seq_len", "jacq_kivi_check_block_table_width",
        "jacq_kivi_decode_workspace_size", "jacq_kivi_decode", "jacq_kivi_cache_append",
        "jacq_kivi_decode_sparse_retained",
        "jacq_kivi_plan_batched_write", "jacq_kivi_profile_start", "jacq_kivi_profile_stop",
        "jacq_kivi_profile_write_ms", "jacq_kivi_profile_wave_stamps", "jacq_kivi_init",
        "jacq_kivi_decode_status", "jacq_kivi_release_workspaces",
        "jacq_kivi_test_device_allocations", "jacq_kivi_write_decode",
        "jacq_kivi_write_decode_workspace_size",
        "jacq_kivi_test_force_merge_timeout", "jacq_kivi_decode_noalloc"])


def test_library_exports_every_declared_function(native):
    missing = [n for n in header_functions() if not hasattr(native, n)]
    assert not missing, missing


def test_jac_launch_argument_order_matches_reference():
    params = header_functions()["jac_launch"]
    assert params == ["Q", "BLOCK_TABLE", "K_CODE_PAGES", "K_SCALE_PAGES", "K_ZERO_PAGES",
                      "V_CODE_PAGES", "V_SCALE_PAGES", "V_ZERO_PAGES", "K_RESIDUAL_SCRATCH",
                      "V_RESIDUAL_SCRATCH", "SEQ_LEN", "O", "stream"]
    order = list(geometry.JAC_LAUNCH_ORDER)
    assert order[:-1] == params[:-1] and order[-1].endswith("stream")
    assert "K_RESIDUAL" not in order and "V_RESIDUAL" not in order
    # source_patch.py:589-595: the dense order with RETAINED_BLOCK_TABLE and
    # NUM_RETAINED_PAGES in place of BLOCK_TABLE and after SEQ_LEN
    sparse = header_functions()["jac_launch_sparse_retained"]
    assert sparse == (["Q", "RETAINED_BLOCK_TABLE"] + params[2:11] + ["NUM_RETAINED_PAGES", "O",
                                                                      "stream"])
    assert header_functions()["jac_launch_sparse_retained_tp2_local"] == sparse
    batched = header_functions()["jac_launch_batched"]
    assert batched[:3] == ["Q", "SEQ_LENS", "BLOCK_TABLE"] and batched[-3:] == [
        "NUM_QUERIES", "O", "stream"]


def test_versions(native):
    assert native.jacq_kivi_abi_version() == abi.JACQ_KIVI_ABI_VERSION == 1
    assert native.jacq_kivi_ext_version() == abi.JACQ_KIVI_EXT_VERSION


def load_probe():
    return json.load(open(os.path.join(ROOT, "tests", "golden", "gpu_boundary_probe.json")))


def test_boundary_probe_python_validator():
    for case in load_probe()["cases"]:
        t = torch.zeros(case["width"], dtype=torch.int32)
        if case["status"] == "accepted":
            kivi.check_block_table_width(t, "BLOCK_TABLE", case["seq_len"])
        else:
            with pytest.raises(kivi.KiviCheckError, match="must be at least"):
                kivi.check_block_table_width(t, "BLOCK_TABLE", case["seq_len"])
    for bad in (0, 4097):  # test_runtime_guards.py:189-197
        with pytest.raises(kivi.KiviCheckError):
            kivi.check_block_table_width(torch.zeros(124, dtype=torch.int32), "BLOCK_TABLE", bad)


def test_boundary_probe_native_validator(native):
    probe = load_probe()
    g = geo(**{k: v for k, v in probe["geometry"].items()})
    for case in probe["cases"]:
        rc = native.jacq_kivi_check_block_table_width(ctypes.byref(g), case["width"],
                                                     case["seq_len"])
        assert (rc == 0) == (case["status"] == "accepted"), case
    for bad in (0, 4097):
        assert native.jacq_kivi_check_block_table_width(ctypes.byref(g), 124, bad) != 0
    assert native.jacq_kivi_max_seq_len(ctypes.byref(g)) == 4096


def test_required_width_every_length(native):
    """The width rule at page 16 and 32 for every length up to the cap:
    floor((L - R) / 32) groups of 32 / P pages."""
    for page in (16, 32):
        g = geo(page_size=page, max_pages_per_seq=124 * 32 // page)
        cap = native.jacq_kivi_max_seq_len(ctypes.byref(g))
        assert cap == 4096
        for L in range(1, cap + 1, 7):
            need = max(0, (L - 128) // 32) * (32 // page)
            assert native.jacq_kivi_check_block_table_width(ctypes.byref(g), need, L) == 0
            if need:
                assert native.jacq_kivi_check_block_table_width(ctypes.byref(g), need - 1, L) != 0


@pytest.mark.parametrize("kw,ok", [
    ({}, True),
    (dict(page_size=16, max_pages_per_seq=248), True),
    (dict(num_heads=20, num_kv_heads=4), True),
    (dict(num_heads=32, num_kv_heads=4, head_dim=64), True),
    (dict(num_heads=14, num_kv_heads=2, head_dim=64, residual=32), True),
    (dict(head_dim=96), False),
    (dict(page_size=8), False),
    (dict(group_size=64), False),
    (dict(residual=100), False),
    (dict(num_heads=40, num_kv_heads=6), False),
    (dict(num_heads=68, num_kv_heads=4), False),  # 17 query heads per kv head
    (dict(num_pages=0), False),
])
def test_geometry_accept_reject(native, kw, ok):
    assert (native.jacq_kivi_check_geometry(ctypes.byref(geo(**kw))) == 0) == ok
    if not ok:
        assert native.jacq_kivi_last_error()


def test_layout_byte_math_matches_reference_fixture():
    """tests/test_layout_and_scaffold.py:162-179 of the reference, at its lane
    geometry (Qwen2.5-Coder-32B: 64 layers, 40/8 heads, HD 128, page 32)."""
    pb = geometry.page_bytes(geometry.V1)
    assert pb["fp16_equivalent"] == 131_072
    assert pb["k_codes"] == 16_384 and pb["v_codes"] == 16_384
    assert pb["k_params"] == 4_096 and pb["v_params"] == 4_096
    assert pb["total"] == 40_960
    assert geometry.V1.residual // geometry.V1.page_size == 4
    assert geometry.stored_bytes_per_token(geometry.V1, 4096, 64) == 87_552.0
    assert 2.99 < geometry.capacity_vs_fp16(geometry.V1, 4096, 64) < 3.0
    with pytest.raises(ValueError, match="straddle"):
        geometry.LaneGeometry(40, 8, 128, page_size=16).require("v1")
    geometry.LaneGeometry(40, 8, 128, page_size=16).require("runtime")
    # page 16: a key group's pairs are stored on both of its pages
    p16 = geometry.page_bytes(geometry.LaneGeometry(40, 8, 128, page_size=16))
    assert p16["k_params"] == 4_096 and p16["k_codes"] == 8_192


def test_launch_argument_table_matches_the_header(native):
    """The Python argument table and include/jacq_kivi.h name the same
    arguments in the same order, and their byte sizes follow the layout."""
    assert list(geometry.JAC_LAUNCH_ORDER[:-1]) == header_functions()["jac_launch"][:-1]
    b = geometry.argument_bytes(geometry.V1, pool_pages=124)
    assert b["K_CODE_PAGES"] == 124 * 16_384 and b["V_SCALE_PAGES"] == 124 * 2_048
    assert b["K_RESIDUAL_SCRATCH"] == 8 * 160 * 128 * 2 and b["O"] == 40 * 128 * 4


def test_decode_bytes_formula():
    """160 bytes per token per kv head at HD=128, 80 at HD=64 (quantised part)."""
    assert geometry.decode_kv_bytes_per_token(128) == 160
    assert geometry.decode_kv_bytes_per_token(64) == 80
    # one sequence of 4096 at the v1 shape: 3968 quantised, 128 fp16 tokens
    n = geometry.decode_step_bytes([4096], 40, 8, 128, 32, 128)
    assert n == 8 * (3968 * 160 + 128 * 512) + 4 * 124 + 40 * 128 * 6


def test_write_step_bytes_formula():
    """The fused step's writer bytes: the new K and
    V rows per sequence, and per age-out 2*32*HD*2 rows in, codes, the K and V
    scale/zero pairs and the R-row shift read and written, per kv head."""
    assert geometry.write_step_bytes([1000, 3000], 8, 128, 128) == 2 * 8 * 512  # no age-out
    per_head = 2 * 32 * 128 * 2 + 2 * 32 * 64 + 128 * 4 + 32 * 4 * 4 + 2 * 2 * 128 * 256
    # 159 -> 160 and 191 -> 192 age a group out, 160 -> 161 does not
    assert geometry.write_step_bytes([159, 160, 191], 8, 128, 128) == 3 * 8 * 512 + 2 * 8 * per_head


def plan_count_closed_form(start, num, residual, group):
    """Sub-chunks of the greedy plan (source_patch.py:521-546), from the
    arithmetic alone: the first takes the room left in the scratch,
    cap - res0; each later one starts from a residual of exactly R (a full
    scratch of R + 32 rows just aged one group out) and takes one group."""
    old0 = max(0, start - residual) // group * group
    room0 = residual + group - (start - old0)
    return 1 if num <= room0 else 1 + -(-(num - room0) // group)


def check_plan(plan, start, num, residual, group):
    cap = residual + group
    seq = start
    assert len(plan) == plan_count_closed_form(start, num, residual, group)
    for idx, (s0, n, scratch_start, page, post) in enumerate(plan):
        assert s0 == seq and n >= 1
        old = max(0, s0 - residual) // group * group
        assert scratch_start == s0 - old
        assert scratch_start + n <= cap, "a sub-chunk must fit the scratch"
        if idx < len(plan) - 1:
            # greedy: take = min(remaining, room), so every sub-chunk but
            # the last fills the scratch to its capacity
            assert scratch_start + n == cap, "a non-final sub-chunk must fill the scratch"
        else:
            assert n == start + num - s0
        new_old = max(0, s0 + n - residual) // group * group
        assert new_old - old in (0, group), "at most one age-out per sub-chunk"
        if new_old > old:
            assert page == old // group and post == s0 + n - new_old
        else:
            assert page is None and post is None
        seq += n
    assert seq == start + num


@pytest.mark.parametrize("residual,group", [(128, 32), (32, 32), (64, 32)])
def test_plan_batched_write_invariants_and_oracle(native, oracle, residual, group):
    rng = np.random.default_rng(residual)
    cases = [(0, 1), (0, 160), (0, 161), (159, 2), (160, 1), (127, 300), (4000, 96)]
    cases += [(int(a), int(b)) for a, b in zip(rng.integers(0, 5000, 60), rng.integers(1, 700, 60))]
    for start, num in cases:
        plan = kivi.plan_batched_write(start, num, residual, group)
        check_plan(plan, start, num, residual, group)
        assert plan == oracle.plan_batched_write(start, num, residual, group)


def _mutant_planner(start, num, residual, group, kind):
    """Plausible mistakes in the planner: an off-by-one room, a take of one
    group at a time, and room counted from the residual window alone."""
    cap = residual + group
    plan, seq, rem = [], start, num
    while rem > 0:
        old = max(0, seq - residual) // group * group
        res = seq - old
        room = {"room-1": cap - res - 1, "group": group, "residual": residual - res}[kind]
        take = min(rem, max(room, 1))
        new_old = max(0, seq + take - residual) // group * group
        aged = new_old > old
        plan.append((seq, take, res, old // group if aged else None,
                     seq + take - new_old if aged else None))
        seq += take
        rem -= take
    return plan


@pytest.mark.parametrize("kind", ["room-1", "group", "residual"])
def test_plan_check_rejects_mutant_planners(kind):
    """check_plan pins the exact cut: each mutant fails it on some case the
    real planners pass."""
    caught = 0
    for start, num in [(0, 1), (0, 160), (0, 161), (159, 2), (127, 300), (4000, 96), (10, 500)]:
        try:
            check_plan(_mutant_planner(start, num, 128, 32, kind), start, num, 128, 32)
        except AssertionError:
            caught += 1
    assert caught > 0


def test_plan_closed_form_small_brute_force():
    """The count formula against a direct simulation of the scratch (append
    until it holds R + 32 rows, then age one group out) on all small inputs."""
    for residual, group in ((32, 32), (64, 32), (128, 32)):
        cap = residual + group
        for start in range(0, 3 * cap):
            for num in range(1, 3 * cap):
                res = start - max(0, start - residual) // group * group
                chunks, left = 0, num
                while left:
                    t = min(left, cap - res)
                    chunks += 1
                    left -= t
                    res += t
                    if res == cap:
                        res -= group
                assert chunks == plan_count_closed_form(start, num, residual, group)


def test_plan_batched_write_rejects_like_reference(native):
    for start, num in ((-1, 4), (0, 0), (3, -2)):
        with pytest.raises(ValueError):
            kivi.plan_batched_write(start, num)


def _compile(tmp_path, name, src, cmd):
    import subprocess
    f = tmp_path / name
    f.write_text(src)
    r = subprocess.run(cmd[:1] + [str(f)] + cmd[1:], capture_output=True, text=True, cwd=tmp_path)
    assert r.returncode == 0, r.stderr[-3000:]


def test_header_compiles_as_c(tmp_path):
    _compile(tmp_path, "c_user.c", '#include "jacq_kivi.h"\nint main(void){return jacq_kivi_abi_version() - 1;}\n',
             ["gcc", "-std=c99", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT}/include",
              "-I/opt/rocm/include"])


def test_reference_style_cxx_binding_links(tmp_path):
    """A translation unit declaring the writer entry points exactly as the
    reference binding does (source_patch.py:570-658, hipified types) links
    against the library: C symbols by name, the two C++ ones by mangled name."""
    src = r'''
#include <hip/hip_runtime_api.h>
#include <hip/hip_fp16.h>
#include <cstdint>
extern "C" void jac_launch(const __half* Q, const int* BLOCK_TABLE,
    const unsigned char* K_CODE_PAGES, const __half* K_SCALE_PAGES, const __half* K_ZERO_PAGES,
    const unsigned char* V_CODE_PAGES, const __half* V_SCALE_PAGES, const __half* V_ZERO_PAGES,
    const __half* K_RESIDUAL_SCRATCH, const __half* V_RESIDUAL_SCRATCH,
    int SEQ_LEN, float* O, hipStream_t stream);
extern "C" void jac_launch_sparse_retained(const __half* Q, const int* RETAINED_BLOCK_TABLE,
    const unsigned char* K_CODE_PAGES, const __half* K_SCALE_PAGES, const __half* K_ZERO_PAGES,
    const unsigned char* V_CODE_PAGES, const __half* V_SCALE_PAGES, const __half* V_ZERO_PAGES,
    const __half* K_RESIDUAL_SCRATCH, const __half* V_RESIDUAL_SCRATCH,
    int SEQ_LEN, int NUM_RETAINED_PAGES, float* O, hipStream_t stream);
void kivi_cache_write_launch(unsigned char* K_CODE_PAGES, __half* K_SCALE_PAGES,
    __half* K_ZERO_PAGES, unsigned char* V_CODE_PAGES, __half* V_SCALE_PAGES,
    __half* V_ZERO_PAGES, __half* K_RESIDUAL_SCRATCH, __half* V_RESIDUAL_SCRATCH,
    const __half* NEW_K, const __half* NEW_V, const int64_t* SLOT_MAPPING,
    const int* BLOCK_TABLE, int seq_len, int NKV_RUNTIME, hipStream_t stream);
void kivi_cache_write_batched_launch(unsigned char* K_CODE_PAGES, __half* K_SCALE_PAGES,
    __half* K_ZERO_PAGES, unsigned char* V_CODE_PAGES, __half* V_SCALE_PAGES,
    __half* V_ZERO_PAGES, __half* K_RESIDUAL_SCRATCH, __half* V_RESIDUAL_SCRATCH,
    const __half* NEW_K, const __half* NEW_V, const int64_t* SLOT_MAPPING,
    const int* BLOCK_TABLE, int START_SEQ_LEN, int NUM_NEW, int NKV_RUNTIME, hipStream_t stream);
int main(int argc, char**) {
  if (argc > 99) {  // referenced, never called: no GPU work on the CPU
    jac_launch(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
               nullptr, 0, nullptr, nullptr);
    jac_launch_sparse_retained(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                               nullptr, nullptr, nullptr, 0, 0, nullptr, nullptr);
    kivi_cache_write_launch(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                            nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, nullptr);
    kivi_cache_write_batched_launch(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                    nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0,
                                    0, nullptr);
  }
  return 0;
}
'''
    lib_dir = os.path.dirname(kivi.library_path())
    _compile(tmp_path, "binding.cpp", src,
             ["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-o",
              str(tmp_path / "binding"), f"-L{lib_dir}", "-ljacq_kivi", "-Wl,--no-as-needed",
              f"-Wl,-rpath,{lib_dir}", "-L/opt/rocm/lib", "-lamdhip64"])


def test_runtime_entry_points_reject_unaligned_pointers(native):
    """Both runtime entry points refuse a base address that is not 16-byte
    aligned before any HIP call (the kernels move 16-byte vectors)."""
    g = geo()
    ok, odd = 1 << 20, (1 << 20) + 2
    decode = [ok] * 11
    decode[0] = odd  # Q offset by one fp16 element
    assert native.jacq_kivi_decode(ctypes.byref(g), *decode, 1, ok, None, 0, None) == 1
    assert b"16-byte aligned" in native.jacq_kivi_last_error()
    append = [ok] * 12
    append[8] = odd  # NEW_K
    assert native.jacq_kivi_cache_append(ctypes.byref(g), *append, 1, 1, None) == 1
    assert b"16-byte aligned" in native.jacq_kivi_last_error()


def test_sparse_retained_entry_point_rejects_like_reference(native):
    """The runtime sparse-retained entry point applies the reference op's
    NUM_RETAINED_PAGES / SEQ_LEN checks (source_patch.py:942-945) before any
    HIP call."""
    g = geo()  # 124-entry table, 1000 pages
    ok = 1 << 20
    caches = [ok] * 8

    def call(seq_len, retained):
        return native.jacq_kivi_decode_sparse_retained(ctypes.byref(g), ok, seq_len, ok,
                                                       retained, *caches, ok, None, 0, None)
    for seq_len, retained, msg in ((4096, -1, b"NUM_RETAINED_PAGES"),
                                   (4096, 125, b"NUM_RETAINED_PAGES"),
                                   (0, 3, b"SEQ_LEN"), (124 * 32 + 129, 3, b"SEQ_LEN")):
        assert call(seq_len, retained) == 1
        assert msg in native.jacq_kivi_last_error()
    small = geo(num_pages=10)
    assert native.jacq_kivi_decode_sparse_retained(ctypes.byref(small), ok, 4096, ok, 11,
                                                   *caches, ok, None, 0, None) == 1
    assert b"physical page storage" in native.jacq_kivi_last_error()


def test_build_spill_guard_parses_resource_remarks():
    """The build rejects a stream / writer kernel that spills (scratch makes the
    decode ~13% slower); the guard reads the compiler's resource remarks."""
    from jacq_amd import build as b
    remarks = "\n".join([
        "x.hip:1:1: remark: Function Name: _ZN4jacq25kivi_decode_stream_kernelILi128ELi16ELb1EEEvNS_7KiviGeoENS_10DecodeArgsE [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     VGPRs: 161 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 12 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     Occupancy [waves/SIMD]: 3 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark: Function Name: _ZN4jacq18kivi_append_kernelENS_7KiviGeoENS_10AppendArgsE [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     VGPRs: 90 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
    ])
    r = b.kernel_resources(remarks)
    stream = [v for k, v in r.items() if "kivi_decode_stream_kernel" in k][0]
    assert stream == {"vgprs": 161, "scratch": 12, "occupancy": 3}
    append = [v for k, v in r.items() if "kivi_append_kernel" in k][0]
    assert append["scratch"] == 0
