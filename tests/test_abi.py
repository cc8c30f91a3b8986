"""CPU checks of the C-ABI library and the host logic: the shared library loads,
exports every entry point the headers declare, and its pure (device-free)
functions behave as the reference's callers expect. No compute call is made."""
import ctypes
import glob
import os
import re
import subprocess

import numpy as np
import pytest

from open_rknpu2_lm_infer_amd import _ffi as F
from open_rknpu2_lm_infer_amd import npu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for path in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(rk_npu_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib_path = F.LIB_PATH
    assert os.path.exists(lib_path), "build the library first"
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    declared = declared_functions()
    assert len(declared) > 60
    missing = sorted(declared - exported)
    assert not missing, f"declared but not exported: {missing}"
    assert set(F.SIGNATURES) == declared, "ctypes table and headers disagree"
    L = F.lib()
    for name in declared:
        assert hasattr(L, name)


def test_headers_compile_as_c():
    src = "".join(f'#include "{os.path.basename(h)}"\n' for h in sorted(glob.glob(os.path.join(ROOT, "include", "*.h"))))
    src += "int main(void) { return 0; }\n"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                    "-x", "c", "-"], input=src, text=True, check=True)


def test_strerror_and_codes():
    assert F.strerror(0) == "success"
    assert F.strerror(F.RK_NPU_ERR_CACHE_MISS) == "tuning cache miss"
    assert F.strerror(12345) == "unknown error"


def test_k_partition_query_table():
    """src/npu.rs:1568-1595 (legality the caller's W8 planning relies on)."""
    L = F.lib()
    for rows, k, tile in [(1, 8192, 2752), (4, 8192, 2752), (64, 8192, 2048), (64, 8192, 3072),
                          (64, 8192, 4096), (64, 6144, 3072), (64, 2560, 2560), (64, 5120, 4096)]:
        assert L.rk_npu_matmul_k_partition_query(rows, k, tile) == 0
    for rows, k, tile in [(64, 8192, 2752), (5, 8192, 2752), (64, 3840, 3840), (64, 3840, 4096),
                          (0, 8192, 4096), (64, 8192, 0)]:
        assert L.rk_npu_matmul_k_partition_query(rows, k, tile) == F.RK_NPU_ERR_PARAM


def test_queries_and_config_init_without_a_device():
    L = F.lib()
    req = F.rk_npu_matmul_weight_requirements()
    assert L.rk_npu_f32i8f32_weights_memory_query(ctypes.byref(F.rk_npu_matmul_weight_config(2560, 9728, 2560)),
                                                  ctypes.byref(req)) == 0
    assert req.bytes == 2560 * 9728 + 9728 * 4
    nb = ctypes.c_uint64()
    assert L.rk_npu_i4_weights_memory_query(ctypes.byref(F.rk_npu_i4_weight_config(2560, 19456, 0)),
                                            ctypes.byref(nb)) == 0
    assert nb.value == 2560 * 19456 // 2 + 19456 * 4
    cfg = F.rk_npu_w4a8_config()
    L.rk_npu_w4a8_config_init(ctypes.byref(cfg), 128, 19456, 2560)
    assert (cfg.M, cfg.N, cfg.K, cfg.m_tile, cfg.n_tile) == (128, 19456, 2560, 64, 1024)
    info = F.rk_npu_w4a8_memory_info_ex()
    opt = F.rk_npu_w4a8_options()
    L.rk_npu_w4a8_options_init(ctypes.byref(opt))
    assert L.rk_npu_w4a8_memory_query_ex(ctypes.byref(cfg), ctypes.byref(opt), ctypes.byref(info)) == 0
    assert info.workspace_bytes > 128 * 2560
    at = F.rk_npu_matmul_autotune_config()
    L.rk_npu_matmul_autotune_config_init(ctypes.byref(at), 1, 256, 256)
    s1, s2 = F.rk_npu_matmul_strategy(), F.rk_npu_matmul_strategy()
    assert L.rk_npu_matmul_autotune_cache_load(None, b"/nonexistent", F.RK_NPU_MATMUL_F32I8F32_DYNAMIC,
                                               ctypes.byref(at), ctypes.byref(s1),
                                               ctypes.byref(s2)) == F.RK_NPU_ERR_CACHE_MISS
    mc = F.rk_npu_moe_w8_config()
    L.rk_npu_moe_w8_config_init(ctypes.byref(mc), 2048, 768, 128, 0, 8, 512)
    assert (mc.weights.hidden, mc.weights.intermediate, mc.weights.routed_experts, mc.top, mc.max_rows) == \
        (2048, 768, 128, 8, 512)


def test_documented_switches_exist():
    """Every plan switch rk_npu_hip.h documents is one rk_npu_hip_set_switch
    knows (set to its current value and restored); unknown names fail."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = open(os.path.join(root, "include", "rk_npu_hip.h")).read()
    block = text[text.index("Plan switches for tests and measurements"):text.index("int rk_npu_hip_set_switch")]
    names = re.findall(r"^ \*   (HM_[A-Z0-9_]+)\s", block, re.M)
    assert len(names) >= 10
    L = F.lib()
    for name in names:
        prev = ctypes.c_int()
        assert L.rk_npu_hip_set_switch(name.encode(), 0, ctypes.byref(prev)) == 0, name
        assert L.rk_npu_hip_set_switch(name.encode(), prev.value, None) == 0, name
    assert L.rk_npu_hip_set_switch(b"HM_NO_SUCH_SWITCH", 1, None) == F.RK_NPU_ERR_PARAM
    # and every switch of the library's table is documented
    src = open(os.path.join(root, "open_rknpu2_lm_infer_amd", "csrc", "hip_matmul.hip")).read()
    table = src[src.index("static const SwitchDef kSwitches"):]
    table = table[:table.index("};")]
    assert set(re.findall(r'"(HM_[A-Z0-9_]+)"', table)) == set(names)


def test_plans():
    L = F.lib()
    plan = F.rk_npu_hip_plan()
    # decode rows run the GEMV on 8-column weight tiles
    assert L.rk_npu_hip_linear_plan(1, 2560, 19456, 4, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n, plan.k_splits, plan.grid) == (0, 1, 8, 1, 19456 // 8)
    assert L.rk_npu_hip_linear_plan(8, 2560, 6144, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m) == (0, 8)
    # 2 to 8 rows need K_pad % 128 == 0 (W8) or % 256 (W4) for the GEMV's
    # matrix-core dots; other K take the GEMM
    assert L.rk_npu_hip_linear_plan(4, 640, 768, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m) == (0, 4)
    assert L.rk_npu_hip_linear_plan(4, 640, 768, 4, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n) == (1, 32, 128)
    assert L.rk_npu_hip_linear_plan(1, 640, 768, 4, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m) == (0, 1)
    assert L.rk_npu_hip_linear_plan(4, 768, 768, 4, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m) == (0, 4)
    # a K too long for the GEMV's quantized rows in LDS (8 x 9728 bytes) takes the GEMM
    assert L.rk_npu_hip_linear_plan(8, 9728, 2560, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n) == (1, 32, 128)
    # 64x128 tiles up to 1024 rows, then 128x128; above 2048 rows 256x256 for
    # very wide outputs and for long K once 128x128 tiles overflow two per CU;
    # K split in pieces when the tiles leave CUs idle and K is long (256 CUs
    # assumed without a GPU): above 256 rows on the 128x128 tile, as many
    # pieces as one round of blocks holds; up to 256 rows on 64x128
    assert L.rk_npu_hip_linear_plan(512, 9728, 2560, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n, plan.k_splits, plan.grid) == (1, 128, 128, 3, 4 * 20 * 3)
    assert L.rk_npu_hip_linear_plan(256, 9728, 2560, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n, plan.k_splits, plan.grid) == (1, 64, 128, 5, 4 * 20 * 5)
    assert L.rk_npu_hip_linear_plan(512, 4096, 2560, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n, plan.k_splits, plan.grid) == (1, 64, 128, 1, 8 * 20)
    assert L.rk_npu_hip_linear_plan(2048, 9728, 2560, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n, plan.k_splits, plan.grid) == (1, 128, 128, 1, 16 * 20)
    assert L.rk_npu_hip_linear_plan(4096, 2560, 9728, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n, plan.k_splits) == (1, 128, 128, 1)
    assert L.rk_npu_hip_linear_plan(4096, 2560, 151936, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n, plan.k_splits) == (1, 256, 256, 1)
    assert L.rk_npu_hip_linear_plan(4096, 9728, 2560, 8, ctypes.byref(plan)) == 0
    # (192x256 where it takes fewer rows per CU: 22 x 10 tiles in one round of
    # 256 CUs instead of 16 x 10 of 256 rows)
    assert (plan.kind, plan.block_m, plan.block_n, plan.k_splits, plan.grid) == (1, 192, 256, 1, 22 * 10)
    assert L.rk_npu_hip_linear_plan(3072, 9728, 2560, 8, ctypes.byref(plan)) == 0
    assert (plan.kind, plan.block_m, plan.block_n, plan.k_splits, plan.grid) == (1, 128, 128, 1, 24 * 20)
    assert L.rk_npu_hip_linear_plan(0, 2560, 9728, 8, ctypes.byref(plan)) == F.RK_NPU_ERR_PARAM


def test_open_without_gpu_returns_null_or_context():
    L = F.lib()
    ctx = L.rk_npu_open(b"999")
    assert not ctx  # no such ordinal on any box
    assert not L.rk_npu_iommu_domain_create(None, 0)
    assert not L.rk_npu_w4a8_weights_create(None, ctypes.byref(F.rk_npu_i4_weight_config(8, 8, 0)), None, None)


def test_host_mirror_logic():
    """src/npu.rs:1442-1466 (validate) and the bucket rule."""
    assert [npu.bucket(r) for r in (1, 2, 3, 5, 9, 17, 65, 128, 129, 192, 193, 256)] == \
        [1, 2, 4, 8, 16, 32, 128, 128, 192, 192, 256, 256]
    for bad in (0, 257):
        with pytest.raises(npu.NpuError):
            npu.bucket(bad)
    for bits in (4, 8):
        m = npu.QuantMatrix(bits, 64, 128, np.zeros(64 * 128, np.int8), np.ones(128, np.float32))
        m.validate()
        m.codes = m.codes[:-1]
        with pytest.raises(npu.NpuError):
            m.validate()
        m.codes = np.zeros(64 * 128, np.int8)
        m.scales = np.ones(0, np.float32)
        with pytest.raises(npu.NpuError):
            m.validate()
        m.scales = np.ones(129, np.float32)
        with pytest.raises(npu.NpuError):
            m.validate()
        m.scales = np.ones(128, np.float32)
        m.k = 2**64
        with pytest.raises(npu.NpuError):
            m.validate()
    with pytest.raises(npu.NpuError):
        npu.QuantMatrix(3, 1, 1, np.zeros(1, np.int8), np.ones(1, np.float32)).validate()


def test_router_mirror_matches_oracle():
    from oracle import oracle
    g = np.random.default_rng(3)
    for _ in range(20):
        logits = g.standard_normal(128).astype(np.float32)
        ids, w = npu.routes(logits, 8)
        oi, ow = oracle.routes(logits, 8)
        assert ids == oi.tolist()
        assert np.allclose(w, ow, rtol=0, atol=2e-7)


# ---- the binding surface the reference's unchanged crate needs -----------------

# Constants whose Rust type the reference's code fixes outside a field or
# argument: error codes compared with i32 return codes (src/npu.rs:195,
# 1592, 1778, src/npu/floating.rs:197), the blob version returned as u32
# (src/npu/moe.rs:283-285), the domain count compared with a u32 id
# (src/npu.rs:484).
TYPED_CONSTANTS = {"RK_NPU_ERR_PARAM": "i32", "RK_NPU_ERR_CACHE_MISS": "i32",
                   "RK_NPU_MOE_QUANT_BLOB_VERSION": "u32", "RK_NPU_IOMMU_DOMAIN_COUNT": "u32"}


@pytest.fixture(scope="module")
def headers():
    from tests import c_abi_model
    if c_abi_model.clang() is None:
        pytest.skip("no clang to parse the headers")
    return c_abi_model.Headers()


@pytest.fixture(scope="module")
def uses():
    import json
    return json.load(open(os.path.join(ROOT, "tests", "golden", "reference_ffi_uses.json")))


def test_headers_declare_every_identifier_the_reference_uses(headers, uses):
    """Every rk_npu_* / RK_NPU_* name the reference's src/ takes from its
    bindings (build.rs:138-158 headers, src/npu.rs and src/npu/*.rs users,
    extracted by tests/golden/extract_ffi_uses.py) is declared here, and the
    four non-hot headers build.rs:141-144 names exist."""
    for h in ("rk_npu_quant_matmul.h", "rk_npu_w4a8_tune.h", "rk_npu_attention_f16.h", "rk_npu_mla_f16.h",
              "rk_npu_mm_tune.h", "rk_npu_mm_gelu.h", "rk_npu_gdn.h", "rk_npu_moe_w8.h"):
        assert os.path.exists(os.path.join(ROOT, "include", h)), h
    missing = sorted(set(uses["identifiers"]) - headers.declared_names())
    assert not missing, f"used by the reference, not declared: {missing}"


def test_struct_fields_the_reference_reads_and_writes_exist(headers, uses):
    missing = [(t, f) for t, f in uses["fields"] if headers.field_type(t, f) is None]
    assert not missing, f"fields the reference's Rust code uses but the headers lack: {missing}"


def test_call_arity_matches_the_reference_call_sites(headers, uses):
    bad = {name: (len(headers.functions[name][1]), arities) for name, arities in uses["call_arity"].items()
           if name in headers.functions and len(headers.functions[name][1]) not in arities}
    assert not bad, f"parameter counts differ from the reference's calls: {bad}"
    assert set(uses["call_arity"]) <= set(headers.functions)


def test_constants_have_the_rust_type_of_their_fields_and_parameters(headers, uses):
    """bindgen types a non-negative #define u32 and an enumerator as its enum's
    underlying type, so `cfg.field = RK_NPU_X` (and ==) only compiles when the
    field's Rust type is that type; the same for a constant passed as an
    argument."""
    bad = []
    for t, f, const, _ in uses["field_constants"]:
        ft, ct = headers.rust_type(headers.field_type(t, f)), headers.constant_type(const)
        if ft != ct:
            bad.append((t, f, ft, const, ct))
    for field, const, _ in uses["named_field_constants"]:
        ct = headers.constant_type(const)
        for rec_name, rec in headers.records.items():
            if rec and field in rec and headers.rust_type(rec[field]) != ct:
                bad.append((rec_name, field, headers.rust_type(rec[field]), const, ct))
    for fn, idx, const in uses["constant_arguments"]:
        pt, ct = headers.rust_type(headers.functions[fn][1][idx]), headers.constant_type(const)
        if pt != ct:
            bad.append((fn, idx, pt, const, ct))
    for const, want in TYPED_CONSTANTS.items():
        if headers.constant_type(const) != want:
            bad.append((const, headers.constant_type(const), want))
    assert not bad, f"constant / field type mismatches bindgen would reject: {bad}"


def test_free_functions_take_one_mutable_handle(headers, uses):
    """Handle<T> keeps `free: unsafe extern "C" fn(*mut T)` (src/npu.rs:163-166)."""
    for name in uses["identifiers"]:
        if name.endswith("_free") and name in headers.functions:
            ret, params = headers.functions[name]
            assert ret == "void" and len(params) == 1 and headers.rust_type(params[0]).startswith("*mut "), name


def test_non_hot_entry_points_report_unsupported_without_a_device():
    """The stubs create nothing and say so: a creator returns
    RK_NPU_ERR_UNSUPPORTED and leaves its out-pointer NULL, config_init
    fills defaults, free accepts NULL."""
    L = F.lib()
    out = ctypes.c_void_p(1)
    assert L.rk_npu_mm_plan_create(None, None, ctypes.byref(out)) == F.RK_NPU_ERR_UNSUPPORTED and not out.value
    out = ctypes.c_void_p(1)
    assert L.rk_npu_mla_f16_weights_create(None, None, ctypes.byref(out)) == F.RK_NPU_ERR_UNSUPPORTED
    assert not out.value
    out = ctypes.c_void_p(1)
    assert L.rk_npu_gdn_prepare(None, None, ctypes.byref(out)) == F.RK_NPU_ERR_UNSUPPORTED and not out.value
    out = ctypes.c_void_p(1)
    assert L.rk_npu_mm_gelu_prepare(None, None, ctypes.byref(out)) == F.RK_NPU_ERR_UNSUPPORTED and not out.value
    assert L.rk_npu_mm_autotune_cache_load(None, ctypes.c_void_p(1), None, None, None) == F.RK_NPU_ERR_CACHE_MISS
    assert L.rk_npu_mla_f16_run(None, None, None, None, None, 1, 0, None, None, None) == F.RK_NPU_ERR_UNSUPPORTED
    cfg = (ctypes.c_int32 * 32)()
    L.rk_npu_gdn_config_init(cfg, 64)
    assert cfg[0] == 64
    for name in ("rk_npu_mm_plan_free", "rk_npu_mm_workspace_free", "rk_npu_mla_f16_cache_free",
                 "rk_npu_gdn_workspace_free", "rk_npu_mm_gelu_free", "rk_npu_mm_tuned_weights_free"):
        getattr(L, name)(None)
