"""Static checks of the product tree (no GPU): no compiler shims, no CPU path.

In the spirit of the reference's ``scripts/verify_stage2_5_no_compiler.py:1-24``
(AST-parse the runtime files, forbid ``torch.compile`` / Triton there), widened
to what this build promises: the package contains no tracing compiler, no
Triton, no CUDA/HIP dual code paths, and nothing in it reaches the oracle,
which is test infrastructure only.
"""
import ast
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "lich_amd"
PY_FILES = sorted(p for p in PKG.rglob("*.py") if "_build" not in p.parts)
NATIVE_FILES = sorted(list((PKG / "csrc").glob("*.hip")) + list((PKG / "csrc").glob("*.h"))
                      + list((ROOT / "include").glob("*.h")))


def _code_without_comments_py(path):
    tree = ast.parse(path.read_text(), filename=str(path))
    return tree


@pytest.mark.parametrize("path", PY_FILES, ids=lambda p: str(p.relative_to(ROOT)))
def test_python_parses_and_uses_no_compiler_or_oracle(path):
    tree = _code_without_comments_py(path)
    for node in ast.walk(tree):
        if isinstance(node, ast.Import):
            names = [a.name for a in node.names]
        elif isinstance(node, ast.ImportFrom):
            names = [node.module or ""]
        else:
            names = []
        for n in names:
            root = n.split(".")[0]
            assert root not in ("triton", "oracle", "tilelang"), f"{path}: imports {n}"
        if isinstance(node, ast.Attribute) and node.attr == "compile":
            base = node.value
            assert not (isinstance(base, ast.Name) and base.id == "torch"), f"{path}: torch.compile"
        if isinstance(node, ast.Attribute) and node.attr in ("_dynamo", "jit") and isinstance(node.value, ast.Name) \
                and node.value.id == "torch":
            raise AssertionError(f"{path}: torch.{node.attr}")


def _strip_c_comments(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


@pytest.mark.parametrize("path", NATIVE_FILES, ids=lambda p: str(p.relative_to(ROOT)))
def test_native_sources_have_one_code_path(path):
    code = _strip_c_comments(path.read_text())
    for token in ("__CUDA_ARCH__", "__CUDACC__", "__HIP_PLATFORM_AMD__", "__HIP_PLATFORM_NVIDIA__",
                  "__HIP_PLATFORM_HCC__", "cuda_runtime", "cudaStream", "hipify", "__NVCC__"):
        assert token not in code, f"{path.name}: {token}"
    # every conditional compilation directive is an include guard or a
    # compile-time tuning default, never a platform switch
    for line in code.splitlines():
        s = line.strip()
        if s.startswith(("#if", "#elif")):
            assert re.match(r"#(ifndef|ifdef|if|elif)\s+!?\s*(defined\s*\(?\s*)?(IPC_|WIDE_|RES_|S16_|__cplusplus)", s), \
                f"{path.name}: unexpected conditional {s!r}"


def test_only_the_allowed_places_reach_the_oracle():
    """tests/, __graft_entry__.smoke() and bench.py's CPU baseline may import
    the oracle; no product module may."""
    for path in PY_FILES:
        assert "from oracle" not in path.read_text() and "import oracle" not in path.read_text(), path
    bench = ast.parse((ROOT / "bench.py").read_text())
    users = []
    for fn in [n for n in ast.walk(bench) if isinstance(n, ast.FunctionDef)]:
        for node in ast.walk(fn):
            if isinstance(node, ast.ImportFrom) and (node.module or "").startswith("oracle"):
                users.append(fn.name)
    assert set(users) <= {"cpu_baseline"}, users
    entry = ast.parse((ROOT / "__graft_entry__.py").read_text())
    for fn in [n for n in entry.body if isinstance(n, ast.FunctionDef)]:
        uses = any(isinstance(n, ast.ImportFrom) and (n.module or "").startswith("oracle") for n in ast.walk(fn))
        assert not uses or fn.name == "smoke", fn.name


def test_build_targets_gfx950_only():
    text = (PKG / "build.py").read_text()
    assert 'ARCH = "gfx950"' in text and "--offload-arch" in text
    assert "-packed-fp32-ops" in text


def test_only_the_cli_uses_the_cpu_reference_api():
    """lich_amd.reference (the reference's pure-PyTorch API) serves the CLI's
    reference command and the tuner's correctness probe; no training or
    kernel module calls it."""
    for path in PY_FILES:
        if path.name in ("reference.py", "cli.py", "autotune.py"):
            continue
        text = path.read_text()
        assert "from .reference" not in text and "lich_amd.reference" not in text, path


@pytest.mark.parametrize("path", NATIVE_FILES, ids=lambda p: str(p.relative_to(ROOT)))
def test_native_sources_allocate_no_device_memory(path):
    """The library allocates nothing: every buffer comes from the caller (plan
    workspaces, the standalone calls' optional workspace) or is the static
    scratch of the no-allocation entry point.  No allocating HIP routine, pool
    or host-pinning call appears in any native source."""
    code = _strip_c_comments(path.read_text())
    for token in ("hipMalloc", "hipFree", "hipMemPool", "hipExtMalloc", "hipHostMalloc", "hipHostRegister",
                  "hipMallocManaged", "hipMemCreate", "hipMemAddressReserve"):
        assert token not in code, f"{path.name}: {token}"
