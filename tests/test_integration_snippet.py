"""The op-level binding that INTEGRATION.md shows a maintainer adding to a
ggml backend (its first C++ block: to_qwm and qwm_try_mul_mat_id; and the
gate/up/SwiGLU node fusion, qwm_try_gate_up_swiglu) compiles against the
reference's own ggml.h and include/qwmoe.h, and the layouts it
relies on hold there: the ggml_type values the C ABI names equal ggml's,
GGML_MAX_DIMS is 4, and qwm_tensor's ne/nb arrays match ggml_tensor's.
Skipped where the reference tree is absent."""
import os
import re
import subprocess

import pytest

from tests.helpers import ROOT

GGML_INC = "/root/reference/third_party/ggml/include"

CHECKS = r"""
static_assert(GGML_MAX_DIMS == 4, "qwm_tensor carries four dimensions");
static_assert(GGML_TYPE_F32 == QWM_TYPE_F32 && GGML_TYPE_Q8_0 == QWM_TYPE_Q8_0 && GGML_TYPE_Q4_K == QWM_TYPE_Q4_K &&
              GGML_TYPE_Q5_K == QWM_TYPE_Q5_K && GGML_TYPE_Q6_K == QWM_TYPE_Q6_K && GGML_TYPE_I32 == QWM_TYPE_I32,
              "ggml_type values");
static_assert(sizeof(((ggml_tensor *)0)->ne) == sizeof(((qwm_tensor *)0)->ne), "ne[]");
static_assert(sizeof(((ggml_tensor *)0)->nb) == sizeof(((qwm_tensor *)0)->nb), "nb[]");
static_assert(sizeof(((ggml_tensor *)0)->ne[0]) == sizeof(int64_t) && sizeof(((ggml_tensor *)0)->nb[0]) == sizeof(size_t),
              "element types of ne[] and nb[]");
// the stub is used, so the snippet's functions are instantiated and checked
bool use_snippet(ggml_tensor * node, void * ws, size_t n, hipStream_t s) { return qwm_try_mul_mat_id(node, ws, n, s); }
int use_fusion(ggml_tensor ** nodes, int n, void * ws, size_t b, hipStream_t s) { return qwm_try_gate_up_swiglu(nodes, n, 0, ws, b, s); }
"""


def snippet():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```cpp\n(.*?)```", text, re.S)
    block = next(b for b in blocks if "qwm_try_mul_mat_id" in b and "to_qwm" in b)
    fusion = next(b for b in blocks if "qwm_try_gate_up_swiglu" in b)
    return block + fusion


@pytest.mark.skipif(not os.path.isdir(GGML_INC), reason="the reference tree is not present")
def test_integration_snippet_compiles_against_ggml(tmp_path):
    src = tmp_path / "binding.cpp"
    src.write_text('#include <hip/hip_runtime_api.h>\n#include "ggml.h"\n' + snippet() + CHECKS)
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                        "-I/opt/rocm/include", "-I" + GGML_INC, "-I" + os.path.join(ROOT, "include"), str(src)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
