# SPDX-License-Identifier: BSD-3-Clause
"""Build of libxtc_hip.so (gfx950) and libxtc_hip_pmu.so (host code, GPU
counters through rocprofiler-sdk).

The GEMM/conv kernel template (gemm.hpp) is instantiated for the tile
configurations listed by `instances()`; the instances are spread over several
generated translation units compiled in parallel, plus a registry unit that
concatenates their entry tables.  Everything lands in-tree:
  xtc_amd/_build/   generated sources and objects
  xtc_amd/lib/libxtc_hip.so
  xtc_amd/lib/libxtc_hip_pmu.so

Usage: python -m xtc_amd.csrc.build [-j JOBS] [-v]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
ROOT = PKG.parent
BUILD = PKG / "_build"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libxtc_hip.so"
PMU_LIB = LIBDIR / "libxtc_hip_pmu.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
INCLUDE = ROOT / "include"

ARCH = "gfx950"
# Packed fp32 VALU forms are kept out of every HIP object.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

F32, BF16 = 0, 1
LDS_LIMIT = 160 * 1024


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return path


def tile_legal(dtype: int, conv: int, bm: int, bn: int, bk: int, wgm: int, wgn: int) -> bool:
    """Mirrors the static_asserts of GemmTile in gemm.hpp."""
    f32 = dtype == F32
    vec = 4 if f32 else 8
    esize = 4 if f32 else 2
    nt = wgm * wgn * 64
    if bm % (16 * wgm) or bn % (16 * wgn):
        return False
    if bk % (16 if f32 else 32):
        return False
    a_chunks = bm * (bk // vec)
    if a_chunks % nt and a_chunks > nt:
        return False
    b_units = bk * (bn // 4) if f32 else (bk // 8) * (bn // 8)
    if b_units % nt and b_units > nt:
        return False
    return lds_bytes(dtype, bm, bn, bk) <= LDS_LIMIT


def lds_bytes(dtype: int, bm: int, bn: int, bk: int) -> int:
    f32 = dtype == F32
    vec = 4 if f32 else 8
    esize = 4 if f32 else 2
    a = bm * (bk + vec)
    b = bk * (bn + 4) if f32 else bn * (bk + 8)
    return 2 * (a + b) * esize


def instances() -> list[tuple[int, int, int, int, int, int, int]]:
    """(dtype, conv, bm, bn, bk, wgm, wgn) of every compiled kernel."""
    out: list[tuple[int, int, int, int, int, int, int]] = []
    waves = [(1, 1), (2, 2), (1, 4), (4, 1), (2, 4), (4, 2)]
    for dtype in (F32, BF16):
        bks = (16, 32) if dtype == F32 else (32, 64)
        for bm in (16, 32, 64, 128, 256):
            for bn in (32, 64, 128, 256):
                for bk in bks:
                    for wgm, wgn in waves:
                        wtm, wtn = bm // wgm, bn // wgn
                        if wtm < 16 or wtn < 16:
                            continue
                        # 8-wave groups only for the largest block tiles
                        if wgm * wgn == 8 and bm * bn < 128 * 256:
                            continue
                        # single-wave groups only for small block tiles
                        if wgm * wgn == 1 and bm * bn > 64 * 64:
                            continue
                        # accumulator registers per lane (fp32)
                        if wtm * wtn // 64 > 256:
                            continue
                        # fp32 256x256 slabs of 32 exceed the register file
                        if dtype == F32 and bm * bn == 256 * 256 and bk == 32:
                            continue
                        # keep wave tiles within a 4:1 aspect ratio
                        if max(wtm, wtn) > 4 * min(wtm, wtn) and min(wtm, wtn) > 16:
                            continue
                        if tile_legal(dtype, 0, bm, bn, bk, wgm, wgn):
                            out.append((dtype, 0, bm, bn, bk, wgm, wgn))
    # fp32 128x128x32 with 8 waves (2x4 of 64x32): the LDS-DMA fp32 kernel's
    # tile for N-narrow GEMMs (runtime.hip routes aligned shapes to it)
    if tile_legal(F32, 0, 128, 128, 32, 2, 4) and (F32, 0, 128, 128, 32, 2, 4) not in out:
        out.append((F32, 0, 128, 128, 32, 2, 4))
    # implicit-GEMM conv loaders: the conv shapes have small N (= F channels)
    for dtype in (F32, BF16):
        bk = 32 if dtype == F32 else 64
        for bm, bn, wgm, wgn in [
            (32, 64, 1, 2),
            (64, 32, 2, 1),
            (64, 64, 2, 2),
            (64, 64, 1, 1),
            (128, 64, 2, 2),
            (128, 64, 4, 1),
            (128, 128, 2, 2),
            (256, 64, 4, 1),
            (256, 128, 2, 2),
            (32, 32, 1, 1),
            (64, 128, 2, 2),
        ]:
            for bkk in ((16, 32) if dtype == F32 else (32, 64)):
                if tile_legal(dtype, 1, bm, bn, bkk, wgm, wgn):
                    out.append((dtype, 1, bm, bn, bkk, wgm, wgn))
    return sorted(set(out))


def ring_tile(dtype: int, conv: int, bm: int, bn: int, bk: int, wgm: int, wgn: int) -> bool:
    """Tiles that also get a ring-3 instance (three register sets of global
    loads in flight, pipeline depth 4): the 64x64 tiles that default_tile
    picks, with split-K, for few tiles over a deep K."""
    return (bm, bn, wgm, wgn) == (64, 64, 2, 2) and bk in ((16, 32) if dtype == F32 else (32, 64))


def _ctype(dtype: int) -> str:
    return "float" if dtype == F32 else "__bf16"


def generate(parts: int = 16) -> list[Path]:
    BUILD.mkdir(parents=True, exist_ok=True)
    insts = instances()
    chunks: list[list[tuple]] = [[] for _ in range(parts)]
    for i, inst in enumerate(insts):
        chunks[i % parts].append(inst)
    files = []
    for p, chunk in enumerate(chunks):
        lines = [
            "// generated by xtc_amd/csrc/build.py -- do not edit",
            '#include "registry.hpp"',
            "namespace xtc_hip {",
        ]
        for dtype, conv, bm, bn, bk, wgm, wgn in chunk:
            c = "true" if conv else "false"
            for ring in (1, 3) if ring_tile(dtype, conv, bm, bn, bk, wgm, wgn) else (1,):
                lines.append(
                    f"template __global__ void gemm_kernel<{_ctype(dtype)}, {bm}, {bn}, {bk}, "
                    f"{wgm}, {wgn}, {c}, {ring}>(GemmArgs);"
                )
        lines += ["#if !defined(__HIP_DEVICE_COMPILE__)", f"extern const GemmEntry g_gemm_part{p}[] = {{"]
        for dtype, conv, bm, bn, bk, wgm, wgn in chunk:
            c = "true" if conv else "false"
            r = "true" if ring_tile(dtype, conv, bm, bn, bk, wgm, wgn) else "false"
            lines.append(
                f"  make_entry<{_ctype(dtype)}, {bm}, {bn}, {bk}, {wgm}, {wgn}, {c}, {r}>(),"
            )
        if not chunk:
            lines.append("  GemmEntry{-1, -1, 0, 0, 0, 0, 0, 0, 0, nullptr, nullptr},")
        lines += [
            "};",
            f"extern const int g_gemm_part{p}_n = {len(chunk)};",
            "#endif",
            "}  // namespace xtc_hip",
            "",
        ]
        f = BUILD / f"gemm_part{p}.hip"
        _write_if_changed(f, "\n".join(lines))
        files.append(f)
    reg = [
        "// generated by xtc_amd/csrc/build.py -- do not edit",
        '#include "registry.hpp"',
        "#include <vector>",
        "#if !defined(__HIP_DEVICE_COMPILE__)",
        "namespace xtc_hip {",
    ]
    for p in range(parts):
        reg.append(f"extern const GemmEntry g_gemm_part{p}[];")
        reg.append(f"extern const int g_gemm_part{p}_n;")
    reg += [
        "const GemmEntry* gemm_registry(int* count) {",
        "  static const std::vector<GemmEntry> all = [] {",
        "    std::vector<GemmEntry> v;",
    ]
    for p in range(parts):
        reg.append(
            f"    for (int i = 0; i < g_gemm_part{p}_n; ++i) v.push_back(g_gemm_part{p}[i]);"
        )
    reg += [
        "    return v;",
        "  }();",
        "  *count = (int)all.size();",
        "  return all.data();",
        "}",
        "}  // namespace xtc_hip",
        "#endif",
        "",
    ]
    f = BUILD / "gemm_registry.hip"
    _write_if_changed(f, "\n".join(reg))
    files.append(f)
    return files


def _write_if_changed(path: Path, text: str) -> None:
    if path.exists() and path.read_text() == text:
        return
    path.write_text(text)


def _compile(src: Path, obj: Path, verbose: bool) -> tuple[Path, float]:
    cmd = [
        hipcc(),
        *HIPCC_FLAGS,
        f"-I{CSRC}",
        f"-I{INCLUDE}",
        "-c",
        str(src),
        "-o",
        str(obj),
    ]
    t0 = time.time()
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr[-6000:]}")
    return obj, time.time() - t0


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compiles every kernel instance and links in-tree libxtc_hip.so."""
    t0 = time.time()
    srcs = [CSRC / "runtime.hip", *generate()]
    objs = [BUILD / (s.stem + ".o") for s in srcs]
    jobs = jobs or max(1, min(16, os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, verbose) for s, o in zip(srcs, objs)]
        for f in futs:
            obj, dt = f.result()
            if verbose:
                print(f"  {obj.name}: {dt:.1f}s", flush=True)
    LIBDIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-shared",
        "-fPIC",
        "-o",
        str(tmp),
        *map(str, objs),
    ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIB)
    build_pmu(verbose)
    if verbose:
        print(f"built {LIB} ({len(instances())} kernel instances) in {time.time() - t0:.1f}s")
    return LIB


def build_pmu(verbose: bool = False) -> Path:
    """libxtc_hip_pmu.so: plain C++ against rocprofiler-sdk (no device code)."""
    LIBDIR.mkdir(parents=True, exist_ok=True)
    tmp = PMU_LIB.with_suffix(".so.tmp")
    cmd = [
        shutil.which("g++") or "g++",
        "-std=c++17",
        "-O2",
        "-fPIC",
        "-shared",
        f"-I{ROCM / 'include'}",
        f"-I{INCLUDE}",
        str(CSRC / "pmu.cpp"),
        f"-L{ROCM / 'lib'}",
        "-lrocprofiler-sdk",
        f"-Wl,-rpath,{ROCM / 'lib'}",
        "-o",
        str(tmp),
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"libxtc_hip_pmu build failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, PMU_LIB)
    return PMU_LIB


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--list", action="store_true", help="print the instance list")
    args = ap.parse_args(argv)
    if args.list:
        for inst in instances():
            print(inst)
        print(len(instances()), "instances")
        return 0
    build(args.jobs, args.verbose)
    return 0


if __name__ == "__main__":
    sys.exit(main())
