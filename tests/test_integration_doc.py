"""The integration guide's call sites compile against the real headers.

Every ```cpp block of INTEGRATION.md is a piece of code a maintainer adds to
the reference. They are assembled, in document order, into one translation
unit: the reference's own `struct Tensor` (src/tensor/tensor.hpp:17-121,
read where it lies) with the `tensor-fields` block added as members of a
local struct of that name, then include/qlm_hip.h and include/qlm_engine.h,
then the other blocks. `g++ -fsyntax-only -Wall -Werror` must accept it, so
a signature change in either header breaks this test instead of the guide.
Skipped where the reference tree is absent (it is only read here).
"""

import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_TENSOR = "/root/reference/src/tensor/tensor.hpp"


def blocks():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    return re.findall(r"^```cpp([^\n]*)\n(.*?)^```", text, flags=re.M | re.S)


def test_guide_has_blocks():
    kinds = [k.strip() for k, _ in blocks()]
    assert kinds.count("tensor-fields") == 1 and len(kinds) >= 6, kinds


@pytest.mark.skipif(not os.path.exists(REF_TENSOR), reason="reference tree not present")
def test_guide_snippets_compile(tmp_path):
    fields = "".join(body for kind, body in blocks() if kind.strip() == "tensor-fields")
    code = "\n".join(body for kind, body in blocks() if kind.strip() != "tensor-fields")
    tu = f"""#include <stdexcept>
#include <string>
#include <vector>
#define Tensor RefTensor
#include "{REF_TENSOR}"
#undef Tensor
#include "qlm_hip.h"
#include "qlm_engine.h"

struct Tensor : RefTensor {{
    using RefTensor::RefTensor;
{fields}
}};

{code}
"""
    src = tmp_path / "guide.cpp"
    src.write_text(tu)
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror",
                        "-Wno-unused-function", "-I", os.path.join(ROOT, "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
