# SPDX-License-Identifier: Unlicense
"""CPU: the drop-in boundary. The reference's callers of the matcher
networks (matcher_eloftr.c, matcher_roma.c, matcher_disk.c, matcher.c of
i.coregistration.opencl) compile unchanged against this build's include/
headers (ops.h, eloftr.h, roma.h, disk.h, pth_loader.h, ocl_backend.h),
and so do main.c's backend calls (main.c:184-185,720-721,903-906),
restated here as a short C file.

This is a syntax and type check (gcc -fsyntax-only -Wall -Werror), not a
build: nothing is linked or run. The callers include GRASS's gis.h and
glocale.h, which the image lacks; the test writes a prototype header of
the six GRASS functions and two macros they use into its temporary
folder. The callers are read where they lie in /root/reference and
given to gcc on standard input from that folder, where only their own
headers (matcher*.h, adalam.h) are placed, so that `#include "eloftr.h"`
resolves to include/ and not to the reference's copy. Skipped where the
reference is absent (the GPU box)."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF = Path("/root/reference")
CALLERS = ("matcher_eloftr.c", "matcher_roma.c", "matcher_disk.c", "matcher.c")
CALLER_HEADERS = ("matcher.h", "matcher_eloftr.h", "matcher_roma.h", "matcher_disk.h",
                  "adalam.h")

pytestmark = pytest.mark.skipif(not all((REF / f).exists() for f in CALLERS + CALLER_HEADERS),
                                reason="the reference's caller sources are not present")

GRASS_GIS = """\
#include <stddef.h>
#define GPATH_MAX 4096
void *G_malloc(size_t);
void *G_calloc(size_t, size_t);
void *G_realloc(void *, size_t);
void G_free(void *);
void G_debug(int, const char *, ...);
void G_fatal_error(const char *, ...) __attribute__((noreturn));
"""

MAIN_CALLS = """\
#include "ocl_backend.h"
#include "ops.h"

int backend_lifecycle(const char *device, const char *platform)
{
    struct ocl_backend ocl;
    struct ops ops;

    ocl_init(&ocl, device, platform);
    ops_init(&ops, &ocl);
    if (ocl.profile)
        ops_report();
    ops_free(&ops);
    ocl_free(&ocl);
    return 0;
}
"""


@pytest.fixture(scope="module")
def workdir(tmp_path_factory):
    d = tmp_path_factory.mktemp("boundary")
    (d / "grass").mkdir()
    (d / "grass" / "gis.h").write_text(GRASS_GIS)
    (d / "grass" / "glocale.h").write_text("#define _(s) (s)\n")
    for h in CALLER_HEADERS:
        shutil.copy(REF / h, d / h)
    return d


def syntax_check(workdir, name, text):
    """gcc -fsyntax-only on text given on standard input, from workdir: a
    quoted include then searches workdir first (not the reference's
    folder), then include/."""
    cmd = ["gcc", "-fsyntax-only", "-Wall", "-Werror", "-std=gnu11", f"-I{workdir}",
           f"-I{ROOT / 'include'}", "-x", "c", "-"]
    p = subprocess.run(cmd, input=text, capture_output=True, text=True, cwd=workdir)
    assert p.returncode == 0, f"{name}:\n{p.stderr}"


@pytest.mark.parametrize("caller", CALLERS)
def test_reference_caller_compiles_unchanged(workdir, caller):
    syntax_check(workdir, caller, (REF / caller).read_text())


def test_main_backend_calls_compile(workdir):
    syntax_check(workdir, "main_calls.c", MAIN_CALLS)


def test_headers_are_the_ones_checked(workdir):
    """The callers' own folder holds none of the headers this build
    replaces, so the check above read include/'s versions."""
    for h in ("ops.h", "eloftr.h", "roma.h", "disk.h", "pth_loader.h", "ocl_backend.h"):
        assert not (workdir / h).exists()
        assert (ROOT / "include" / h).exists()
