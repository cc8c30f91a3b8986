"""The drop-in as the reference crate's build script builds and links it (CPU
tests, no GPU).

build.rs:52-74 configures the CMake project at RK_NPU_MATMUL_ROOT (this
repository) with -DCMAKE_BUILD_TYPE=Release -DBUILD_TESTING=OFF
-DRK_NPU_ENABLE_TRACE=OFF and builds the target rk_npu_matmul_static;
build.rs:76-94 builds the crate's own CPU kernels (native/cpu_kernels:
swiglu.cpp, gdn.cpp, kda.cpp, with "${RK_NPU_MATMUL_ROOT}/src" on the include
path); build.rs:89-130 links librknpu2_cpu_kernels.a, librk_npu_matmul.a,
the OpenMP libraries named by OpenMP_CXX_LIB_NAMES / OpenMP_<name>_LIBRARY in
the CMake cache, then stdc++, pthread, m and dl. The one change a maintainer
makes is adding the HIP runtime (amdhip64) to that list.

Here: the CMake target is built as build.rs builds it; the CPU kernels are
compiled from the crate's sources with g++ and the flags of
native/cpu_kernels/CMakeLists.txt:3-22 (C++17 with GNU extensions, -Wall
-Wextra -Werror, PIC, OpenMP); one C translation unit takes the address of
every function the crate calls (the bindgen-bound rk_npu_* calls extracted
from the crate's sources into tests/golden/reference_ffi_uses.json, and the
crate's own extern blocks: src/npu.rs:63-66, src/model/cpu.rs:87-89,
src/ops/gated_delta/native.rs:22-25, src/ops/kda.rs:76-78,
src/ops/gelu.rs:3-5) and is linked with exactly that link line plus
amdhip64. The link must leave no symbol unresolved.

The reference's checkout is read here (its CPU kernel sources); without it
the tests that need it are skipped."""
import json
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_CPU_KERNELS = "/root/reference/native/cpu_kernels"
BUILD = os.path.join(ROOT, "tests", "dropin", "_build")
ROCM_LIB = "/opt/rocm/lib"

BINDGEN_HEADERS = ["rk_npu_quant_matmul.h", "rk_npu_w4a8_tune.h", "rk_npu_attention_f16.h", "rk_npu_mla_f16.h",
                   "rk_npu_mm_tune.h", "rk_npu_mm_gelu.h", "rk_npu_gdn.h", "rk_npu_moe_w8.h"]  # build.rs:138-145

# The crate's extern "C" declarations outside bindgen, as C prototypes
# (trace hooks only exist with cfg(rknpu_trace), which the default build
# leaves off: src/model/trace.rs:5-11).
CRATE_EXTERNS = {
    "omp_set_dynamic": "void omp_set_dynamic(int);",
    "omp_set_num_threads": "void omp_set_num_threads(int);",
    "rknpu2_cpu_swiglu": "void rknpu2_cpu_swiglu(const float*, const float*, float*, size_t);",
    "rknpu2_gdn_run": "void rknpu2_gdn_run(const void*);",
    "rknpu2_gdn_run_unfused": "void rknpu2_gdn_run_unfused(const void*);",
    "rknpu2_kda_run": "void rknpu2_kda_run(const void*);",
    "erff": "float erff(float);",
}


def tool(name):
    path = shutil.which(name) or (os.path.join("/opt/rocm/bin", name) if os.path.exists(
        os.path.join("/opt/rocm/bin", name)) else None)
    if not path:
        pytest.skip(f"{name} is not available")
    return path


def run(cmd, **kw):
    res = subprocess.run(cmd, capture_output=True, text=True, **kw)
    assert res.returncode == 0, f"{' '.join(cmd)}\n{res.stdout[-4000:]}\n{res.stderr[-4000:]}"
    return res


def cmake_cache(path):
    values = {}
    for line in open(path):
        if "=" in line and not line.startswith(("//", "#")):
            entry, value = line.rstrip("\n").split("=", 1)
            values[entry.split(":", 1)[0]] = value
    return values


def openmp_libraries(build_dir):
    """build.rs:6-28: the OpenMP libraries the CMake cache names, resolved."""
    cache = cmake_cache(os.path.join(build_dir, "CMakeCache.txt"))
    libs = []
    for name in cache["OpenMP_CXX_LIB_NAMES"].split(";"):
        path = cache[f"OpenMP_{name}_LIBRARY"]
        assert os.path.exists(path), path
        libs.append(os.path.realpath(path))
    return libs


@pytest.fixture(scope="module")
def native_build():
    """build.rs:60-74: configure and build rk_npu_matmul_static (the HIP
    sources compile in parallel; later runs are incremental)."""
    cmake = tool("cmake")
    tool("hipcc")
    out = os.path.join(BUILD, "native")
    os.makedirs(out, exist_ok=True)
    run([cmake, "-S", ROOT, "-B", out, "-DCMAKE_BUILD_TYPE=Release", "-DBUILD_TESTING=OFF",
         "-DRK_NPU_ENABLE_TRACE=OFF"])
    run([cmake, "--build", out, "--target", "rk_npu_matmul_static", "--config", "Release", "-j", "8"])
    return out


def test_static_target_and_openmp_cache(native_build):
    archive = os.path.join(native_build, "librk_npu_matmul.a")
    assert os.path.exists(archive), "build.rs links librk_npu_matmul.a from the top of the build directory"
    libs = openmp_libraries(native_build)
    assert libs and all(os.path.exists(p) for p in libs)
    # the archive's public symbols include every rk_npu_* function the headers declare
    from tests.test_abi import declared_functions
    out = run(["nm", "--defined-only", "-g", archive]).stdout
    defined = {line.split()[-1] for line in out.splitlines() if re.search(r" T ", line)}
    missing = sorted(declared_functions() - defined)
    assert not missing, missing


def cpu_kernels_archive():
    """native/cpu_kernels/CMakeLists.txt:3-22 with g++: swiglu.cpp, gdn.cpp and
    kda.cpp with this repository's src/ on the include path."""
    if not os.path.isdir(REF_CPU_KERNELS):
        pytest.skip("the reference's native/cpu_kernels sources are not present")
    gxx = tool("g++")
    out = os.path.join(BUILD, "cpu_kernels")
    os.makedirs(out, exist_ok=True)
    objs = []
    for src in ("swiglu.cpp", "gdn.cpp", "kda.cpp"):
        obj = os.path.join(out, src.replace(".cpp", ".o"))
        run([gxx, "-std=gnu++17", "-O3", "-DNDEBUG", "-fPIC", "-fopenmp", "-Wall", "-Wextra", "-Werror",
             "-I", os.path.join(ROOT, "src"), "-c", os.path.join(REF_CPU_KERNELS, src), "-o", obj])
        objs.append(obj)
    archive = os.path.join(out, "librknpu2_cpu_kernels.a")
    if os.path.exists(archive):
        os.remove(archive)
    run(["ar", "rcs", archive, *objs])
    return out


def test_unchanged_crate_links(native_build):
    cpu_dir = cpu_kernels_archive()
    uses = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_ffi_uses.json")))
    called = sorted(uses["call_arity"])
    assert len(called) >= 80
    src = ["#include <stddef.h>", "#include <stdio.h>"]
    src += [f'#include "{h}"' for h in BINDGEN_HEADERS]
    src += list(CRATE_EXTERNS.values())
    names = called + sorted(CRATE_EXTERNS)
    src.append("static void* const refs[] = {")
    src += [f"    (void*)&{n}," for n in names]
    src.append("};")
    src.append("int main(void) {")
    src.append('    printf("%zu\\n", sizeof(refs) / sizeof(refs[0]));')
    src.append("    return 0;")
    src.append("}")
    out = os.path.join(BUILD, "link")
    os.makedirs(out, exist_ok=True)
    c_path = os.path.join(out, "crate_externs.c")
    with open(c_path, "w") as f:
        f.write("\n".join(src) + "\n")
    cc = tool("gcc")
    obj = os.path.join(out, "crate_externs.o")
    run([cc, "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), "-c", c_path, "-o", obj])
    # build.rs:89-130, in its order, plus amdhip64
    link = [cc, obj, "-o", os.path.join(out, "crate_externs"),
            "-L", cpu_dir, "-lrknpu2_cpu_kernels",
            "-L", native_build, "-lrk_npu_matmul"]
    assert openmp_libraries(native_build)  # build.rs asserts both caches agree; one compiler here
    for lib in openmp_libraries(native_build):
        link += ["-L", os.path.dirname(lib), f"-l:{os.path.basename(lib)}"]
    link += ["-lstdc++", "-lpthread", "-lm", "-ldl", "-L", ROCM_LIB, "-lamdhip64", f"-Wl,-rpath,{ROCM_LIB}"]
    res = subprocess.run(link, capture_output=True, text=True)
    assert res.returncode == 0, f"unresolved at link:\n{res.stderr[-6000:]}"
    undefined = run(["nm", "-u", os.path.join(out, "crate_externs")]).stdout
    for n in names:
        assert not re.search(rf"\bU {re.escape(n)}$", undefined, re.M), n


def test_swiglu_header_matches_the_library_arithmetic(tmp_path):
    """src/rk_npu_swiglu_fp32_neon.h computes bit for bit what the library's
    SwiGLU epilogues compute (the oracle's orc_swiglu, which the GPU parity
    tests hold the kernels to), for the 16-wide call of
    native/cpu_kernels/swiglu.cpp:13-21, including the +-80 saturation, the
    signed-zero tail and the optional row max; compiled with the contraction
    GCC allows by default for C++ (-ffp-contract=fast), as the crate's CPU
    kernels are."""
    gxx = tool("g++")
    test = tmp_path / "swiglu_check.cpp"
    test.write_text(r'''
#include "rk_npu_swiglu_fp32_neon.h"
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
extern "C" float orc_swiglu(float gate, float up);
static uint32_t bits(float v) { uint32_t b; std::memcpy(&b, &v, 4); return b; }
int main() {
    using rknpu2_matmul_open::detail::swiglu_fp32::apply16;
    uint64_t s = 0x5EED;
    auto next = [&]() { s = s * 6364136223846793005ull + 1442695040888963407ull; return (uint32_t)(s >> 32); };
    long bad = 0, n = 0;
    const float special[] = {0.0f, -0.0f, 80.0f, -80.0f, 80.000008f, -80.000008f, 79.99999f, -79.99999f,
                             1e-38f, -1e-38f, 88.0f, -88.0f, 1e30f, -1e30f, 0.5f, -0.5f};
    for (int it = 0; it < 200000; ++it) {
        alignas(16) float g[16], u[16], y[16];
        for (int i = 0; i < 16; ++i) {
            if (it == 0) g[i] = special[i];
            else {
                const float r = (float)(next() >> 8) * (1.0f / 16777216.0f);
                g[i] = (it % 3 == 0) ? (r - 0.5f) * 200.0f : (r - 0.5f) * 16.0f;
            }
            u[i] = ((float)(next() >> 8) * (1.0f / 16777216.0f) - 0.5f) * 8.0f;
        }
        const float mx = apply16<true>(g, u, y);
        float want_mx = 0.0f;
        for (int i = 0; i < 16; ++i) {
            const float w = orc_swiglu(g[i], u[i]);
            want_mx = std::fmax(want_mx, std::fabs(w));
            bad += bits(y[i]) != bits(w);
            ++n;
        }
        bad += bits(mx) != bits(want_mx);
        alignas(16) float y2[16];
        bad += apply16<false>(g, u, y2) != 0.0f || std::memcmp(y, y2, sizeof(y)) != 0;
    }
    std::printf("%ld %ld\n", bad, n);
    return bad != 0;
}
''')
    exe = tmp_path / "swiglu_check"
    # the oracle is C: compile it as C, the check as C++
    ocobj = tmp_path / "rk_oracle.o"
    run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-fopenmp", "-c", os.path.join(ROOT, "oracle", "rk_oracle.c"),
         "-o", str(ocobj)])
    run([gxx, "-std=gnu++17", "-O3", "-ffp-contract=fast", "-Wall", "-Wextra", "-Werror",
         "-I", os.path.join(ROOT, "src"), str(test), str(ocobj), "-fopenmp", "-lm", "-o", str(exe)])
    res = run([str(exe)])
    bad, n = map(int, res.stdout.split())
    assert n == 200000 * 16 and bad == 0
