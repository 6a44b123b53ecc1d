"""The drop-in at the kernel ABI, at link level (build container only).

oracle/Makefile's `linkcheck` target compiles the reference's decoder and
CLI (src/*.c, cli/main.c) from its sources under /root/reference and links
them, with ingot minus its kernel objects (kernels.c, generic.c) as an
archive like the reference's libingot.a, against libmynah_hip.so with
--no-undefined. Nothing is run. Checked here:
  * the link succeeds: every symbol the decoder needs is defined;
  * the kernel entry points the decoder calls (src/arch_qwen3.c:46 ingot_matvec,
    :64 ingot_gguf_matvec, :175 ingot_dequant_matrix) are imported from
    libmynah_hip.so and nothing else of ingot's kernel ABI is;
  * no object or archive member linked defines a symbol the library exports
    (no duplicate definitions);
  * the executable exports ingot_gguf_data, which the library's
    ingot_gguf_matvec uses to locate a tensor's bytes;
  * the front-end binding of the generation loop (oracle/generate_hip.c, the
    code a maintainer adds beside src/generate.c) compiles against the
    reference's headers and links: mynah_slm_generate_hip and
    mynah_slm_generate_hip_dev are defined and their loop,
    mynah_hip_qwen3_generate_tokens, comes from the library.
"""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
LIB = os.path.join(ROOT, "mynah-slm_amd", "libmynah_hip.so")
EXE = os.path.join(ROOT, "oracle", "_ref", "mynah-slm-hip")

pytestmark = pytest.mark.skipif(
    not os.path.exists(os.path.join(REF, "src", "arch_qwen3.c")) or not os.path.exists(LIB),
    reason="needs the reference sources (build container) and the built library")


def nm(args):
    out = subprocess.run(["nm"] + args, check=True, capture_output=True, text=True).stdout
    rows = []
    for line in out.splitlines():
        parts = line.split()
        if len(parts) >= 2:
            rows.append((parts[-2], parts[-1]))
    return rows


@pytest.fixture(scope="module")
def linked():
    r = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "linkcheck"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return EXE


def test_decoder_links_with_no_undefined_symbol(linked):
    assert os.path.exists(linked)


def test_kernel_calls_resolve_to_the_library(linked):
    ours = {s for t, s in nm(["-D", "--defined-only", LIB]) if t in "TWiDBR"}
    imported = {s for t, s in nm(["-D", linked]) if t == "U" and s.startswith("ingot_")}
    assert imported == {"ingot_matvec", "ingot_gguf_matvec", "ingot_dequant_matrix"}
    assert imported <= ours
    exported = {s for t, s in nm(["-D", "--defined-only", linked])}
    assert "ingot_gguf_data" in exported


def test_no_linked_object_redefines_a_library_symbol(linked):
    ours = {s for t, s in nm(["-D", "--defined-only", LIB]) if t in "TWiDBR"}
    obj = os.path.join(ROOT, "oracle", "_ref", "obj")
    members = [os.path.join(obj, "dec_src", f) for f in os.listdir(os.path.join(obj, "dec_src"))]
    members += [os.path.join(obj, "dec_cli", "main.o"),
                os.path.join(ROOT, "oracle", "_ref", "libingot_nokern.a")]
    defined = set()
    for m in members:
        defined |= {s for t, s in nm(["--defined-only", m]) if t.isupper()}
    assert not (defined & ours), sorted(defined & ours)


def test_generate_binding_links(linked):
    ours = {s for t, s in nm(["-D", "--defined-only", LIB]) if t in "TWiDBR"}
    imported = {s for t, s in nm(["-D", linked]) if t == "U" and s.startswith("mynah_hip_")}
    assert imported == {"mynah_hip_qwen3_generate_tokens"} and imported <= ours
    assert ("T", "mynah_slm_generate_hip") in set(nm([linked]))
    assert ("T", "mynah_slm_generate_hip_dev") in set(nm([linked]))
