"""CPU-only checks of the product library: it loads, it exports exactly what
include/*.h declares, the identity strings match the reference backend, and
its device code contains no floating-point instruction (the integer-only
contract of theta_v; the reference audits the same for its Rust hot path in
INTEGER_LLM/tests/audit/test_no_float.py).  No kernel is launched here."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[\w\s\*]+?\b(myl_\w+)\s*\(", text, flags=re.M):
            if "MYL_HD" in text[max(0, m.start() - 40):m.start() + 40]:
                continue  # header-only inline helpers of myl_synth.h
            names.add(m.group(1))
    return names


def exported_symbols(lib: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if l.split() and l.split()[-1].startswith("myl_")}


def test_library_exports_every_declared_symbol():
    from myelith_amd import _lib
    lib = _lib.LIB_PATH
    assert lib.exists(), "libmyl_hip.so must be built (python -m myelith_amd.build)"
    decl = {n for n in declared_symbols() if not n.startswith("myl_synth") and n not in
            ("myl_mix64", "myl_splitmix_at", "myl_draw_range", "myl_tensor_seed", "myl_ilog2_u64",
             "myl_isqrt_floor")}
    exp = exported_symbols(lib)
    missing = decl - exp
    assert not missing, f"declared but not exported: {sorted(missing)}"
    # the ctypes table covers the same set
    assert decl == set(_lib.SIGNATURES), sorted(decl ^ set(_lib.SIGNATURES))


def test_library_loads_and_names_itself():
    from myelith_amd.backend import RocmBackend
    # rocm.rs:71-82
    assert RocmBackend.name() == "rocm"
    assert RocmBackend.hardware_family() == "amd-gpu"
    assert RocmBackend.feature_tag() == "rocm"


def test_device_code_has_no_floating_point(tmp_path):
    srcs = sorted((ROOT / "myelith_amd" / "csrc").glob("*.hip"))
    assert srcs
    bad = []
    for src in srcs:
        out = tmp_path / (src.stem + ".s")
        r = subprocess.run(["/opt/rocm/bin/hipcc", "-O3", "-std=c++17", "-I", str(ROOT / "include"), "-x", "hip",
                            "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                            "--cuda-device-only", "-S", str(src), "-o", str(out)], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        float_op = re.compile(r"^v_\w*(_f16|_bf16|_f32|_f64|rcp|rsq|sqrt)\w*$")
        for line in out.read_text().splitlines():
            t = line.strip()
            if t.startswith("v_") and float_op.match(t.split()[0]):
                bad.append(f"{src.name}: {t}")
    assert not bad, "floating-point instructions in integer kernels:\n" + "\n".join(bad[:20])


def test_oracle_is_not_linked_into_the_product():
    from myelith_amd import _lib
    out = subprocess.run(["nm", "-D", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    assert " or_" not in out and "liboracle" not in out
    for p in (ROOT / "myelith_amd").rglob("*"):
        if p.suffix in (".py", ".hip", ".cpp", ".h"):
            text = p.read_text()
            assert "oracle" not in text.split("\n", 1)[-1].lower() or p.name == "_lib.py" or "import oracle" not in text, p
            assert "import oracle" not in text and "from oracle" not in text, p
