"""CPU checks of the committed Swift side of the boundary (swift/Libraries):
the CLSamp module map names the library the build produces and an umbrella
header that compiles as C11, and every C function, type and constant the Swift
conformers use is declared by include/lsamp.h.  (swiftc is not in this image,
so the Swift files themselves are not compiled here.)"""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLSAMP = os.path.join(REPO, "swift", "Libraries", "CLSamp")
SWIFT = os.path.join(REPO, "swift", "Libraries", "MLXLMCommon", "LSamp")
HEADER = os.path.join(REPO, "include", "lsamp.h")
LIBDIR = os.path.join(REPO, "mlx-swift-lm_amd", "lib")


def _swift_sources():
    return sorted(os.path.join(SWIFT, f) for f in os.listdir(SWIFT) if f.endswith(".swift"))


def _header_text():
    return re.sub(r"/\*.*?\*/", " ", open(HEADER).read(), flags=re.S)


def test_module_map_names_the_umbrella_header_and_the_library():
    text = open(os.path.join(CLSAMP, "module.modulemap")).read()
    assert re.search(r"\bmodule\s+CLSamp\s+\[system\]", text)
    m = re.search(r'umbrella\s+header\s+"([^"]+)"', text)
    assert m and os.path.isfile(os.path.join(CLSAMP, m.group(1)))
    m = re.search(r'\blink\s+"([^"]+)"', text)
    assert m and m.group(1) == "lsamp"
    # the linker resolves link "lsamp" to liblsamp.so, the file the build writes
    from lsamp import _ffi
    assert os.path.basename(_ffi.LIB_PATH) == "liblsamp.so"


@pytest.mark.parametrize("compiler", ["gcc", "clang"])
def test_umbrella_header_compiles_as_c11(compiler, tmp_path):
    cc = shutil.which(compiler) or (compiler == "clang" and shutil.which("/opt/rocm/llvm/bin/clang"))
    if not cc:
        pytest.skip(f"{compiler} not available")
    src = tmp_path / "use.c"
    src.write_text('#include "CLSamp.h"\n'
                   "int main(void) { lsamp_sample_args a = {0}; (void)a; "
                   "return (int)sizeof(lsamp_step_args) > 0 ? 0 : 1; }\n")
    r = subprocess.run([cc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic",
                        "-fsyntax-only", "-I", CLSAMP, str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_swift_conformers_use_only_declared_c_names():
    header = _header_text()
    declared = set(re.findall(r"\b(lsamp_[a-z0-9_]+)\b", header))
    defined = set(re.findall(r"\b(LSAMP_[A-Z0-9_]+)\b", header))
    used_fn, used_const = set(), set()
    for path in _swift_sources():
        code = re.sub(r"//[^\n]*", " ", open(path).read())
        used_fn |= set(re.findall(r"\b(lsamp_[a-z0-9_]+)\b", code))
        used_const |= set(re.findall(r"\b(LSAMP_[A-Z0-9_]+)\b", code))
    assert used_fn, "the conformers call the C ABI"
    assert not (used_fn - declared), f"not in lsamp.h: {sorted(used_fn - declared)}"
    assert not (used_const - defined), f"not in lsamp.h: {sorted(used_const - defined)}"


def test_swift_conformers_have_no_stubs():
    for path in _swift_sources():
        code = open(path).read()
        assert "fatalError" not in code, f"{os.path.basename(path)} has a fatalError stub"
    names = " ".join(open(p).read() for p in _swift_sources())
    for conformance in ("LogitSampler", "LogitProcessor", "CBv2StepSampler"):
        assert re.search(r":\s*" + conformance + r"\b", names), conformance
