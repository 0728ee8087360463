"""Link compatibility with the reference's callers: its MLA probes and prefill bench
(src/mla_incremental_probe.c, src/spec_q8_lab_probe.c, src/mla_streaming_probe.c,
src/mla_prefill_bench.c) compile against this repository's include/ and link against
libkvl_mla.so. Nothing is run (the programs need a GPU once linked to the library).

The reference keeps src/ops.c in its storage library when the MLA sources are replaced
(CMakeLists.txt:33-34 renames its prefill to kvl_mla_prefill_materialized_bf16, which
mla_streaming_probe.c calls), so that object is built from the reference source and linked
beside the library for that probe, as the reference's link-time selection would."""
import os
import subprocess

import pytest

from kvl_mla import lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SRC = "/root/reference/src"
PROBES = ["mla_incremental_probe", "spec_q8_lab_probe", "mla_streaming_probe", "mla_prefill_bench"]


def _lib_dir():
    if not os.path.exists(lib.LIB_PATH):
        pytest.skip("libkvl_mla.so not built")
    return os.path.dirname(lib.LIB_PATH)


@pytest.fixture(scope="module")
def ops_object(tmp_path_factory):
    if not os.path.isdir(REF_SRC):
        pytest.skip("reference sources not present")
    out = tmp_path_factory.mktemp("ops") / "ops.o"
    subprocess.run(["gcc", "-std=c11", "-O1", "-fopenmp", "-ffunction-sections", "-fdata-sections",
                    "-Dkvl_mla_prefill_bf16=kvl_mla_prefill_materialized_bf16",
                    "-I", os.path.join(os.path.dirname(REF_SRC), "include"),
                    "-c", os.path.join(REF_SRC, "ops.c"), "-o", str(out)], check=True)
    return str(out)


@pytest.mark.parametrize("probe", PROBES)
def test_reference_probe_links_against_library(probe, ops_object, tmp_path):
    libdir = _lib_dir()
    obj = tmp_path / f"{probe}.o"
    exe = tmp_path / probe
    subprocess.run(["gcc", "-std=c11", "-O1", "-I", os.path.join(ROOT, "include"), "-c",
                    os.path.join(REF_SRC, f"{probe}.c"), "-o", str(obj)], check=True)
    undefined = subprocess.run(["nm", "-u", str(obj)], check=True, capture_output=True, text=True).stdout
    needed = sorted({ln.split()[-1] for ln in undefined.splitlines() if ln.split()[-1].startswith("kvl_")})
    exported = subprocess.run(["nm", "-D", "--defined-only", lib.LIB_PATH], check=True,
                              capture_output=True, text=True).stdout
    exported = {ln.split()[-1] for ln in exported.splitlines()}
    from_ops = [s for s in needed if s not in exported]
    # only the materialised prefill may come from ops.c; every other MLA entry is the library's
    assert set(from_ops) <= {"kvl_mla_prefill_materialized_bf16"}, from_ops
    cmd = ["gcc", str(obj)] + ([ops_object] if from_ops else []) + [
        "-fopenmp", "-Wl,--gc-sections", "-Wl,--no-as-needed", "-L", libdir, "-lkvl_mla",
        f"-Wl,-rpath,{libdir}", "-lm", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert exe.exists()
