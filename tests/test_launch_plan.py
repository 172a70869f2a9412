"""The host side of the byte-plane product launches, on the CPU (no GPU).

1. The launch planning (csrc/mm_plan.h: tile counts, the K split, slices,
   work items, grid, LDS) is plain C++ called by the launchers.  Here it is
   built with g++ under AddressSanitizer and UndefinedBehaviorSanitizer
   (every error fatal) and run over every split-K launch shape the dispatch
   uses, for 1-256 activation rows of the 7B and 0.5B products and the
   batched decode's accumulator sizes, checking that the plan covers K and
   the output tiles exactly once, stays within the accumulator, and that
   grid and LDS fit the device.
2. The kernel argument layout the host passes (the launch's argument list,
   laid out by the C ABI rules through ctypes) against the gfx950 code
   object's own metadata (llvm-readelf on the objects this build made), for
   every mm2 kernel instantiation, with the block size and LDS of the launch
   shape.
3. The plans of the fragment-major products of decode batches (the same
   header, gemm_frag.h's launchers) for 1-32 rows on 1-304 CUs, under the
   same sanitizers: K covered, one block per CU, every block's row groups
   within the LDS and the 512 output columns the epilogues map.

Written to look for a host-side cause of an earlier abort inside the
launch sequence of mm2_splitk_kernel<2, 1, 1, 4, 2, 128> (B = 32 batched
decode) under a profiler counter pass.
"""
from __future__ import annotations

import ctypes as C
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "myelith_amd" / "csrc"
BUILD = ROOT / "myelith_amd" / "_build"
LLVM = Path("/opt/rocm/llvm/bin")

# The split-K shapes of gemm_dispatch.h (mm_planes, mm_planes_fin).
SPLIT_SHAPES = [(1, 1, 1, 4, 3, 128), (1, 1, 1, 2, 4, 128), (1, 1, 1, 4, 4, 64), (2, 1, 1, 4, 2, 128),
                (2, 1, 1, 4, 4, 64), (1, 1, 4, 2, 3, 128), (2, 1, 2, 4, 4, 64)]

DRIVER = r"""
#include "mm_plan.h"
#include <cstdio>
#include <cstdlib>
#include <vector>
using namespace myl;
static long checked = 0, bad = 0;
#define CHECK(c, ...) do { ++checked; if (!(c)) { if (bad++ < 20) { std::printf("FAIL " __VA_ARGS__); std::printf("\n"); } } } while (0)

template <int MB, int NB, int WM, int WN, int ST, int KS>
void run(const char* name) {
    using D = Mm2Dims<MB, NB, WM, WN, ST, KS>;
    std::printf("dims %d %d %d %d %d %d threads %d lds %zu\n", MB, NB, WM, WN, ST, KS, D::kThreads, D::kLds);
    CHECK(D::kThreads <= 1024 && D::kThreads % 64 == 0, "%s threads", name);
    CHECK(D::kLds <= 160 * 1024, "%s lds %zu", name, D::kLds);
    // (N, K) of the 7B and 0.5B products on byte planes, K % KS == 0
    const int shapes[][2] = {{4608, 3584}, {3584, 3584}, {37888, 3584}, {3584, 18944}, {152064, 3584},
                             {1152, 896}, {896, 896}, {9728, 896}, {896, 4864}, {151936, 896},
                             {2816, 2048}, {2048, 1408}, {11264, 2048}, {2048, 5632}, {60, 2048}};
    const int cus = 256;
    for (auto& nk : shapes) {
        const int N = nk[0], K = nk[1];
        if (K % KS) continue;
        for (int M = 1; M <= 256; ++M) {
            // the batched forward's accumulator: rows x max(2 I, q/k/v rows); and none
            const size_t accs[] = {(size_t)M * 37888, (size_t)M * (size_t)N, (size_t)M * (size_t)N - 1, 0};
            const int fills[] = {cus / 2, cus, 2 * cus};
            for (size_t acc : accs)
                for (int fill : fills) {
                    const Mm2SplitPlan p = mm2_split_plan<MB, NB, WM, WN, ST, KS>(M, N, K, cus, acc, fill);
                    CHECK(p.tiles_r * D::BR >= 2 * M && (p.tiles_r - 1) * D::BR < 2 * M, "%s M=%d rows", name, M);
                    CHECK(p.ntiles == p.tiles_r * ((N + D::BN - 1) / D::BN), "%s M=%d N=%d tiles", name, M, N);
                    CHECK(p.kslice % KS == 0 && p.kslice > 0, "%s kslice %d", name, p.kslice);
                    CHECK((long)p.ns * p.kslice >= K && (long)(p.ns - 1) * p.kslice < K, "%s M=%d N=%d K=%d slices %d x %d",
                          name, M, N, K, p.ns, p.kslice);
                    CHECK(p.nitems == p.ntiles * p.ns, "%s items", name);
                    CHECK(p.grid >= p.nitems && p.grid % 8 == 0 && p.grid - p.nitems < 8, "%s grid", name);
                    CHECK(p.split == (p.ns > 1) || (p.split && p.ns == 1), "%s split flag", name);
                    if (p.split) {
                        CHECK((size_t)M * (size_t)N <= acc, "%s M=%d N=%d split beyond the accumulator %zu", name, M, N, acc);
                        CHECK(p.ntiles < fill, "%s split with a full grid", name);
                        CHECK(p.kslice >= 512 || p.kslice >= K, "%s slice %d below 512 bytes", name, p.kslice);
                    } else {
                        CHECK(p.kslice == K && p.ns == 1, "%s unsplit slice", name);
                    }
                }
        }
    }
}

int main() {
    run<1, 1, 1, 4, 3, 128>("1,1,1,4,3,128");
    run<1, 1, 1, 2, 4, 128>("1,1,1,2,4,128");
    run<1, 1, 1, 4, 4, 64>("1,1,1,4,4,64");
    run<2, 1, 1, 4, 2, 128>("2,1,1,4,2,128");
    run<2, 1, 1, 4, 4, 64>("2,1,1,4,4,64");
    run<1, 1, 4, 2, 3, 128>("1,1,4,2,3,128");
    run<2, 1, 2, 4, 4, 64>("2,1,2,4,4,64");
    std::printf("checked %ld bad %ld\n", checked, bad);
    return bad != 0;
}
"""


def _gxx():
    return shutil.which("g++")


@pytest.fixture(scope="module")
def plan_run(tmp_path_factory):
    if not _gxx():
        pytest.skip("g++ absent")
    d = tmp_path_factory.mktemp("plan")
    src = d / "driver.cpp"
    src.write_text(DRIVER)
    exe = d / "driver"
    subprocess.run([_gxx(), "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-fno-omit-frame-pointer", "-I", str(CSRC), str(src), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    return r


def test_launch_plan_under_asan_and_ubsan(plan_run):
    r = plan_run
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
    last = r.stdout.strip().splitlines()[-1]
    n = int(re.match(r"checked (\d+) bad 0", last).group(1))
    assert n > 100000


def _dims(plan_run) -> dict:
    out = {}
    for line in plan_run.stdout.splitlines():
        m = re.match(r"dims (\d+) (\d+) (\d+) (\d+) (\d+) (\d+) threads (\d+) lds (\d+)", line)
        if m:
            v = tuple(int(x) for x in m.groups())
            out[v[:6]] = (v[6], v[7])
    return out


def _kernel_notes(tmp_path) -> list[dict]:
    """(name, args [(offset, size, kind)], max threads, static LDS) of every
    kernel in the gfx950 code objects of this build's HIP objects."""
    kernels = []
    for obj in sorted(BUILD.glob("*.hip.o")):
        fat = tmp_path / (obj.stem + ".fat")
        co = tmp_path / (obj.stem + ".co")
        subprocess.run([str(LLVM / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", str(obj)], check=True,
                       capture_output=True)
        subprocess.run([str(LLVM / "clang-offload-bundler"), "--type=o",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={fat}", f"--output={co}",
                        "--unbundle"], check=True, capture_output=True)
        notes = subprocess.run([str(LLVM / "llvm-readelf"), "--notes", str(co)], check=True, capture_output=True,
                               text=True).stdout
        # one kernel entry per "  - .agpr_count" block of amdhsa.kernels
        for blk in re.split(r"\n  - (?=\.agpr_count)", notes)[1:]:
            name = re.search(r"\n    \.name:\s+(\S+)", blk).group(1)
            args = [(int(o), int(s), k) for o, s, k in
                    re.findall(r"\.offset:\s+(\d+)\s*\n\s+\.size:\s+(\d+)\s*\n\s+\.value_kind:\s+(\w+)", blk)]
            threads = int(re.search(r"\.max_flat_workgroup_size:\s+(\d+)", blk).group(1))
            lds = int(re.search(r"\.group_segment_fixed_size:\s+(\d+)", blk).group(1))
            kernels.append(dict(name=name, args=args, threads=threads, lds=lds))
    return kernels


class _Divider(C.Structure):
    """Divider (csrc/gemm_mfma.h): uint32 d, uint64 m."""
    _fields_ = [("d", C.c_uint32), ("m", C.c_uint64)]


def _layout(types) -> list[tuple[int, int]]:
    """Offsets and sizes of a by-value argument list, packed by the C rules."""
    fields = [(f"a{i}", t) for i, t in enumerate(types)]
    S = type("Args", (C.Structure,), {"_fields_": fields})
    return [(getattr(S, f).offset, C.sizeof(t)) for f, t in fields]


P, I32 = C.c_void_p, C.c_int32
# mm2_splitk_kernel(Ap, R2, W, N, K, Divider tiles_r, Divider ntiles, nitems, kslice, acc)
SPLITK_ARGS = [P, I32, P, I32, I32, _Divider, _Divider, I32, I32, P]


@pytest.mark.skipif(not (LLVM / "llvm-readelf").exists(), reason="ROCm LLVM tools absent")
def test_kernel_arguments_match_the_code_object(plan_run, tmp_path):
    if not any(BUILD.glob("*.hip.o")):
        pytest.skip("library not built (myelith_amd/_build)")
    dims = _dims(plan_run)
    kernels = _kernel_notes(tmp_path)
    want = _layout(SPLITK_ARGS)
    seen = 0
    for k in kernels:
        m = re.search(r"mm2_splitk_kernelILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)E", k["name"])
        if not m:
            continue
        shape = tuple(int(x) for x in m.groups())
        explicit = [(o, s) for o, s, kind in k["args"] if not kind.startswith("hidden_")]
        assert explicit == want, (shape, explicit, want)
        threads, lds = dims[shape]
        assert k["threads"] == threads, shape
        assert k["lds"] + lds <= 160 * 1024, shape
        seen += 1
    # every split-K shape the dispatch launches is in the objects
    assert seen >= len(SPLIT_SHAPES)
    assert any(re.search(r"mm2_splitk_kernelILi2ELi1ELi1ELi4ELi2ELi128E", k["name"]) for k in kernels)


FRAG_DRIVER = r"""
#include "mm_plan.h"
#include <cstdio>
using namespace myl;
static long checked = 0, bad = 0, wide = 0;
#define CHECK(c, ...) do { ++checked; if (!(c)) { if (bad++ < 20) { std::printf("FAIL " __VA_ARGS__); std::printf("\n"); } } } while (0)

// the row groups block p of P takes in frag_mm_kernel: [p NG / P, (p + 1) NG / P)
static int block_groups(int p, int P, int NG) { return (int)(((long)(p + 1) * NG) / P - ((long)p * NG) / P); }

int main() {
    // (N, K) of the decode-batch products: gate/up, down, q/k/v, o_proj of the
    // 7B and 0.5B shapes and of the test models (hidden 448 / 4096)
    const int shapes[][2] = {{37888, 3584}, {3584, 18944}, {4608, 3584}, {3584, 3584}, {9728, 896}, {896, 4864},
                             {1152, 896}, {896, 896}, {640, 448}, {448, 320}, {576, 448}, {8320, 4096},
                             {4096, 4160}, {5120, 4096}};
    const int cus_list[] = {1, 2, 3, 4, 7, 8, 16, 32, 38, 64, 80, 128, 160, 256, 304};
    for (int cus : cus_list)
        for (auto& nk : shapes) {
            const int N = nk[0], K = nk[1], KT = K / 64, NG = (N + 15) / 16;
            for (int R = 1; R <= kFragMaxRows; ++R) {
                const int rt = frag_rt(R);
                CHECK(rt == (R <= 8 ? 1 : R <= 16 ? 2 : 4) && 16 * rt >= 2 * R, "rt R=%d", R);
                if (frag_full_ok(R, K, N, cus)) {
                    const int ngb = (NG + cus - 1) / cus, kpw = KT <= kFragWaves * 7 ? 7 : 8;
                    CHECK(kFragWaves * kpw >= KT, "full K=%d cover", K);
                    CHECK(16 * ngb <= kFragWaves * 64, "full N=%d cus=%d width %d", N, cus, 16 * ngb);
                    CHECK(frag_lds(rt, ngb, R, true) <= kFragLdsMax, "full lds");
                    for (int p = 0; p < cus; ++p) CHECK(block_groups(p, cus, NG) <= ngb, "full groups p=%d", p);
                }
                const size_t acc = (size_t)R * (size_t)N;
                const FragSplit sp = frag_split_plan(K, N, cus);
                if (sp.kpw != 0 && 16 * sp.ngb > kFragWaves * 64 && frag_lds(rt, sp.ngb, R, false) <= kFragLdsMax)
                    ++wide;  // plans the column guard turns away
                if (frag_split_ok(R, K, N, cus, acc)) {
                    CHECK(sp.kpw == 8 || sp.kpw == 5, "split kpw %d", sp.kpw);
                    const int span = kFragWaves * sp.kpw;
                    CHECK((long)sp.S * span >= KT && (long)(sp.S - 1) * span < KT, "split K=%d slices %d", K, sp.S);
                    CHECK(sp.S * sp.P <= cus && sp.P >= 1, "split grid %d x %d on %d CUs", sp.S, sp.P, cus);
                    CHECK(sp.ngb == (NG + sp.P - 1) / sp.P && 16 * sp.ngb <= kFragWaves * 64,
                          "split N=%d cus=%d width %d", N, cus, 16 * sp.ngb);
                    CHECK(frag_lds(rt, sp.ngb, R, false) <= kFragLdsMax, "split lds");
                    for (int p = 0; p < sp.P; ++p) CHECK(block_groups(p, sp.P, NG) <= sp.ngb, "split groups p=%d", p);
                    CHECK(!frag_split_ok(R, K, N, cus, acc - 1), "split past the accumulator");
                }
            }
        }
    std::printf("checked %ld bad %ld wide %ld\n", checked, bad, wide);
    return bad != 0;
}
"""


def test_fragment_plans_under_asan_and_ubsan(tmp_path):
    """The fragment-major products' plans (csrc/mm_plan.h) for 1-32 rows of
    every decode-batch product shape on 1-304 CUs: the K slices cover K, the
    grid fits one block per CU, every block's row groups (as the kernel
    splits them) fit the LDS the plan sized and the 512 output columns the
    epilogues map onto the block's threads; plans wider than that exist and
    are turned away."""
    if not _gxx():
        pytest.skip("g++ absent")
    src = tmp_path / "frag.cpp"
    src.write_text(FRAG_DRIVER)
    exe = tmp_path / "frag"
    subprocess.run([_gxx(), "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-fno-omit-frame-pointer", "-I", str(CSRC), str(src), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "runtime error" not in r.stderr
    m = re.match(r"checked (\d+) bad 0 wide (\d+)", r.stdout.strip().splitlines()[-1])
    assert m and int(m.group(1)) > 10000 and int(m.group(2)) > 0, r.stdout[-500:]
