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


def _source(name):
    return open(os.path.join(SWIFT, name)).read()


def _body(code, start):
    """The brace-balanced body of the first declaration matching `start`."""
    m = re.search(start, code)
    assert m, f"no declaration matches {start!r}"
    i = m.end()
    if code[i - 1] == "(":  # skip the parameter list (default values hold braces)
        depth = 1
        while depth:
            depth += {"(": 1, ")": -1}.get(code[i], 0)
            i += 1
    i = code.index("{", i)
    depth = 0
    for j in range(i, len(code)):
        depth += {"{": 1, "}": -1}.get(code[j], 0)
        if depth == 0:
            return code[i:j + 1]
    raise AssertionError(f"unbalanced braces after {start!r}")


# The CBv2StepSampler constraint lifecycle (EngineLoopV2.swift:91-152), as
# its requirements are spelled there: member, then the parameter list.
STEP_SAMPLER_MEMBERS = [
    r"public var supportsTokenConstraints: Bool",
    r"public var supportsConstrainedChainedDecode: Bool",
    r"public func confirmSampledTokens\(_ tokens: \[Int\], requestIDs: \[CBv2RequestID\]\)",
    r"public func tokenConstraintFailure\(for id: CBv2RequestID\) -> String\?",
    r"public func takeInvalidatedChainedRows\(\) -> \[CBv2RequestID\]",
    r"public func redrawChainedSuccessor\(logits: MLXArray, requestIDs: \[CBv2RequestID\]\)"
    r"\s*-> MLXArray\?",
    r"public func requestDidFinish\(_ id: CBv2RequestID\)",
]


@pytest.mark.parametrize("member", STEP_SAMPLER_MEMBERS)
def test_step_sampler_has_the_constraint_lifecycle(member):
    assert re.search(member, _source("LSampStepSampler.swift")), member


def test_step_sampler_claims_constraints_and_masks_on_the_device():
    code = _source("LSampStepSampler.swift")
    for flag in ("supportsTokenConstraints", "supportsConstrainedChainedDecode"):
        assert re.search(r"public var " + flag + r": Bool \{ true \}", code), flag
    # the step's masks are assembled by lsamp_mask_assemble and handed to
    # lsamp_step as the bitmask, with ids past the vocab forbidden
    draw = _body(code, r"func draw\(")
    assert "lsamp_mask_assemble(" in draw and "lsamp_step(" in draw
    assert "st.sample.bitmask" in draw and "LSAMP_MASK_TAIL_FORBID" in draw
    # a speculative sample keeps the table it started from; the redraw
    # restores it and the RNG steps, then draws unspeculatively
    sample = _body(code, r"public func sample\(")
    assert "beginSpeculation()" in sample and "copyTable(toSnapshot: true)" in sample
    redraw = _body(code, r"public func redrawChainedSuccessor\(")
    assert "copyTable(toSnapshot: false)" in redraw and "steps = s.steps" in redraw
    assert "speculative: false" in redraw
    finish = _body(code, r"public func requestDidFinish\(")
    assert "masks.requestDidFinish" in finish
    # the mask bookkeeping mirrors lsamp/constraint.py: confirm, failure and
    # invalidation go through LSampConstraintMasks
    masks = _source("LSampConstraintMasks.swift")
    for fn in ("func configure(", "func plan(", "func confirm(", "func takeInvalidated(",
               "func failure(for", "func requestDidFinish(", "func beginSpeculation("):
        assert fn in masks, fn
    assert "cacheCapacity = 8" in masks


def test_step_sampler_rejects_windows_above_capacity():
    """The repetition window is not clamped to the table's ring: a context
    larger than the ring is a precondition failure, not a shorter window."""
    code = _source("LSampStepSampler.swift")
    configure = _body(code, r"func configure\(_ rows:")
    assert re.search(r"precondition\(\s*!reps \|\| p\.repetitionContextSize <= Int\(windowCapacity\)",
                     configure)
    assert not re.search(r"min\(max\(p\.repetitionContextSize", configure)


def test_outputs_outlive_the_call():
    """Arrays a call returns wrap buffers the sampler owns for its life:
    verify allocates no buffer of its own (a local buffer would be freed
    when the call returns, while the returned arrays still alias it), and
    step outputs rotate through rings."""
    code = _source("LSampStepSampler.swift")
    verify = _body(code, r"func verify\(mode:")
    assert not re.search(r"LSampDeviceBuffer(<[^>]*>)?\(", verify), \
        "verify must not allocate call-local device buffers"
    draw = _body(code, r"func draw\(")
    for ring in ("outTokens.take()", "outFlags.take()", "outChosen.take()"):
        assert ring in draw, ring
    runtime = _source("LSampRuntime.swift")
    assert "final class LSampOutputRing" in runtime
    assert re.search(r"func free\(_ pointer: UnsafeMutableRawPointer\)", runtime)
    assert "ordered on `stream`" in runtime


def test_logit_processor_returns_penalized_logits():
    """LSampLogitProcessor.process returns lsamp_penalize's output unless
    the pair was made with fusedPenalties (SampleTests.swift:431-454: a
    processor after the penalties sees the penalized logits)."""
    code = _source("LSampLogitSampler.swift")
    process = _body(code, r"public func process\(logits: MLXArray\) -> MLXArray")
    assert "if fused { return logits }" in process
    assert "lsamp_penalize(" in process and "logitsArray(" in process
    assert "promotes" in process  # float32 once the frequency window holds a token
    make = _body(code, r"public static func make\(")
    assert "fusedPenalties ? windows : nil" in make
    assert re.search(r"fusedPenalties: Bool = false", code)


def test_logit_sampler_takes_batched_logits():
    code = _source("LSampLogitSampler.swift")
    sample = _body(code, r"public func sample\(logits: MLXArray\) -> MLXArray")
    assert "a.rows = Int32(rows)" in sample
    assert "penalty_row_len" in sample  # one window shared by every row
    rows = _body(code, r"func rows\(_ view:")
    assert "view.shape.count == 2" in rows and "maxRows" in rows


def test_swift_does_not_use_the_test_hooks():
    testing = open(os.path.join(REPO, "include", "lsamp_testing.h")).read()
    hooks = set(re.findall(r"\b(lsamp_test_[a-z0-9_]+)\b", testing))
    assert hooks
    umbrella = " ".join(open(os.path.join(CLSAMP, f)).read()
                        for f in os.listdir(CLSAMP) if f.endswith(".h"))
    assert "lsamp_testing.h" not in umbrella
    for path in _swift_sources():
        assert not (hooks & set(re.findall(r"\b(lsamp_test_[a-z0-9_]+)\b", open(path).read())))
