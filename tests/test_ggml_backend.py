"""The ggml backend plugin (questwend_amd/ggml/ggml-qwmoe.cpp, backend API v3)
builds against the reference's own ggml headers, including the backend
interface header src/ggml-backend-impl.h, with -Wall -Wextra -Werror.

What the built object shows:
  * it exports ggml_backend_init (the symbol ggml_backend_load looks up,
    ggml-backend-reg.cpp:229-237) and ggml_backend_qwmoe_reg;
  * every ggml symbol it leaves undefined is a function that ggml's public or
    backend headers declare, so the process's libggml-base provides it;
  * it needs libqwmoe.so and the HIP runtime, nothing else of ggml.

It is not run here: running it needs libggml-base, whose ggml.c includes a
header that only the reference's CMake generates.  Skipped where the reference
tree is absent."""
import os
import re
import subprocess

import pytest

from tests.helpers import ROOT

GGML = "/root/reference/third_party/ggml"


@pytest.fixture(scope="module")
def plugin(tmp_path_factory):
    if not os.path.isfile(os.path.join(GGML, "src", "ggml-backend-impl.h")):
        pytest.skip("the reference tree is not present")
    if not os.path.isfile(os.path.join(ROOT, "questwend_amd", "libqwmoe.so")):
        pytest.skip("libqwmoe.so is not built")
    out = tmp_path_factory.mktemp("plugin") / "libggml-qwmoe.so"
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "questwend_amd", "ggml"), f"OUT={out}", f"GGML={GGML}"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return str(out)


def symbols(path, *flags):
    r = subprocess.run(["nm", "-D", *flags, path], capture_output=True, text=True, check=True)
    return {line.split()[-1] for line in r.stdout.splitlines() if line.strip()}


def test_plugin_exports_the_backend_entry_points(plugin):
    defined = symbols(plugin, "--defined-only")
    assert {"ggml_backend_init", "ggml_backend_qwmoe_reg"} <= defined
    assert not any(s.startswith("qwm_") for s in defined), "libqwmoe's functions must come from libqwmoe.so"


def test_plugin_needs_only_ggml_base_functions(plugin):
    undefined = symbols(plugin, "-u")
    ggml_syms = sorted(s for s in undefined if s.startswith("ggml_"))
    assert ggml_syms, "the backend calls ggml-base (graph access, buffer init)"
    headers = ""
    for d in (os.path.join(GGML, "include"), os.path.join(GGML, "src")):
        for name in os.listdir(d):
            if name.endswith(".h"):
                headers += open(os.path.join(d, name), errors="replace").read()
    for s in ggml_syms:
        assert re.search(r"GGML_API[^;]*\b" + re.escape(s) + r"\s*\(", headers), f"{s} is not declared by ggml"
    qwm = sorted(s for s in undefined if s.startswith("qwm_"))
    assert "qwm_mul_mat_id" in qwm and "qwm_mul_mat_id_swiglu" in qwm and "qwm_swiglu" in qwm
    exported = symbols(os.path.join(ROOT, "questwend_amd", "libqwmoe.so"), "--defined-only")
    assert set(qwm) <= exported
    r = subprocess.run(["readelf", "-d", plugin], capture_output=True, text=True, check=True)
    needed = re.findall(r"Shared library: \[(.*?)\]", r.stdout)
    assert "libqwmoe.so" in needed and not any(n.startswith("libggml") for n in needed)
