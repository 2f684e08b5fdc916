"""Build recipe of the CPU checkers. TEST INFRASTRUCTURE ONLY.

build_oracle()     gcc -O2 -ffp-contract=off oracle/csrc/oracle.c -> oracle/lib/liboracle.so
build_reference()  the reference's own C++ tree builders, compiled from their sources where they lie
                   under /root/reference (the C++ text embedded in inference/hf/tree_build_ext.py
                   :20-213 and in the SGLang patch's ddtree_utils.py, P:1249-1412), with g++ against
                   torch's headers -> oracle/_ref/ref_hf_builder*.so, oracle/_ref/ref_sglang_builder*.so
                   (Python extension modules). The extracted text goes to a temporary directory that is
                   deleted afterwards; only the compiled modules are kept (oracle/_ref is git-ignored).
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sysconfig
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
REF_DIR = os.path.join(HERE, "_ref")
REFERENCE = "/root/reference"
HF_BUILD_EXT = os.path.join(REFERENCE, "inference", "hf", "tree_build_ext.py")
SGLANG_PATCH = os.path.join(REFERENCE, "inference", "sglang", "patches", "sglang-v0.5.22-mfd.patch")


def build_oracle() -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    out = os.path.join(LIB_DIR, "liboracle.so")
    src = os.path.join(HERE, "csrc", "oracle.c")
    cmd = ["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", src, "-o",
           out + ".tmp", "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(out + ".tmp", out)
    return out


def _new_file_from_patch(patch_path: str, path: str) -> str:
    lines, inside = [], False
    with open(patch_path, encoding="utf-8") as f:
        for line in f:
            if line.startswith("diff --git "):
                inside = line.strip().endswith(f"b/{path}")
                continue
            if inside and line.startswith("+") and not line.startswith("+++"):
                lines.append(line[1:])
    return "".join(lines)


def _cpp_block(text: str) -> str:
    m = re.search(r'_CPP_SOURCE = r"""(.*?)"""', text, re.S)
    if not m:
        raise RuntimeError("no _CPP_SOURCE block found")
    return m.group(1)


def _compile_torch_ext(cpp_text: str, name: str) -> str:
    import torch.utils.cpp_extension as ce

    os.makedirs(REF_DIR, exist_ok=True)
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(REF_DIR, name + suffix)
    tmp = tempfile.mkdtemp(prefix="mfd_ref_")
    try:
        src = os.path.join(tmp, name + ".cpp")
        with open(src, "w") as f:
            f.write(cpp_text)
        incs = [f"-I{p}" for p in ce.include_paths()] + [f"-I{sysconfig.get_paths()['include']}"]
        libdir = os.path.join(os.path.dirname(ce.__file__), "..", "lib")
        import torch

        abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
        cmd = ["g++", "-O3", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
               f"-DTORCH_EXTENSION_NAME={name}", "-DTORCH_API_INCLUDE_EXTENSION_H", *incs, src, "-o", out + ".tmp",
               f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", f"-Wl,-rpath,{os.path.abspath(libdir)}"]
        subprocess.run(cmd, check=True)
        os.replace(out + ".tmp", out)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return out


def _up_to_date(name: str, src: str) -> str | None:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(REF_DIR, name + suffix)
    if os.path.exists(out) and os.path.getmtime(out) >= os.path.getmtime(src):
        return out
    return None


def build_reference(force: bool = False) -> list[str]:
    if not os.path.exists(HF_BUILD_EXT) or not os.path.exists(SGLANG_PATCH):
        raise RuntimeError("/root/reference is not present")
    if not force:
        done = [_up_to_date("ref_hf_builder", HF_BUILD_EXT), _up_to_date("ref_sglang_builder", SGLANG_PATCH)]
        if all(done):
            return done
    outs = []
    with open(HF_BUILD_EXT, encoding="utf-8") as f:
        outs.append(_compile_torch_ext(_cpp_block(f.read()), "ref_hf_builder"))
    sg = _new_file_from_patch(SGLANG_PATCH, "python/sglang/srt/speculative/ddtree_utils.py")
    outs.append(_compile_torch_ext(_cpp_block(sg), "ref_sglang_builder"))
    return outs


if __name__ == "__main__":
    print(build_oracle())
    print(build_reference())
