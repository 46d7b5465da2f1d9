"""CPU checks of the C-ABI boundary: the built library loads, exports every
entry point include/tmopt_attn.h declares, the ctypes table mirrors the
header, and argument validation fails with a status code (no GPU needed:
invalid calls return before any HIP call)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tmopt_attn.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tmopt_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    fns = header_functions()
    for want in ("tmopt_kv_write_slots", "tmopt_kv_write_paged",
                 "tmopt_attn_decode_paged", "tmopt_attn_decode_workspace_size",
                 "tmopt_attn_prefill_varlen", "tmopt_last_error"):
        assert want in fns


def test_library_exports_every_declared_symbol(tm):
    lib = tm._lib.load()
    missing = [f for f in header_functions() if not hasattr(lib, f)]
    assert not missing, missing


def test_ctypes_table_mirrors_header(tm):
    assert sorted(tm._lib.SIGNATURES) == header_functions()


def test_library_symbols_with_nm(tm):
    """The .so's dynamic symbol table carries the C names (no mangling)."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", tm._lib.LIB_PATH],
                         capture_output=True, text=True)
    if out.returncode != 0:
        pytest.skip("nm unavailable")
    names = {l.split()[-1] for l in out.stdout.splitlines() if l.strip()}
    for f in header_functions():
        assert f in names, f


def test_invalid_arguments_return_status(tm):
    lib = tm._lib.load()
    null = ctypes.c_void_p(0)
    # decode: B < 0 is rejected before anything touches the device
    rc = lib.tmopt_attn_decode_paged(null, null, null, null, 1, 0, null, -1,
                                     32, 4, 128, 16, 1, 0, 0.1, null, 0, 8,
                                     0, null, null, null, 0, null)
    assert rc == tm._lib.TMOPT_EINVAL
    assert b"B=-1" in lib.tmopt_last_error()
    # decode: head_dim 64 is outside the supported set
    p = ctypes.c_void_p(16)
    rc = lib.tmopt_attn_decode_paged(p, p, p, p, 1, 0, p, 1, 32, 4, 64, 16,
                                     1, 0, 0.1, null, 0, 8, 0, p, null, p,
                                     1 << 20, null)
    assert rc == tm._lib.TMOPT_EUNSUPPORTED
    # decode: any HQ % HKV == 0 ratio; a prime one above 16 runs as one
    # scheduled KV head per query head, and beyond 65535 of them it is
    # refused
    rc = lib.tmopt_attn_decode_paged(p, p, p, p, 1, 0, p, 1, 17 * 30000,
                                     30000, 128, 16, 1, 0, 0.1, null, 0, 8,
                                     0, p, null, p, 1 << 20, null)
    assert rc == tm._lib.TMOPT_EUNSUPPORTED
    assert b"exceeds 65535" in lib.tmopt_last_error()
    # decode: a ring table of 4 pages (64 positions) with no window, then
    # with a window wider than the ring
    for window in (0, 65):
        rc = lib.tmopt_attn_decode_paged(p, p, p, p, 4, 4, p, 1, 32, 4, 128,
                                         16, 1, window, 0.1, null, 0, 8, 0, p,
                                         null, p, 1 << 20, null)
        assert rc == tm._lib.TMOPT_EINVAL
        assert b"ring of 4 pages" in lib.tmopt_last_error()
    # prefill: any HQ % HKV == 0 ratio; one that would need more than 65535
    # scheduled KV heads (groups of up to 8 query heads) is refused
    rc = lib.tmopt_attn_prefill_varlen(p, 0, 0, p, 0, 0, 0, 1, p, 0, 0,
                                       0, 1, p, null, 1, 4, null, null,
                                       null, 0, 0, 16, 0, 3 * 30000, 30000,
                                       128, 0, 0.1, null, 0, 0, 0, p, 0, 0,
                                       null, null, null)
    assert rc == tm._lib.TMOPT_EUNSUPPORTED
    assert b"exceeds 65535" in lib.tmopt_last_error()

    def prefill(k, prior, table, wrap, window):
        return lib.tmopt_attn_prefill_varlen(
            p, 4096, 128, k, 0, 512, 128, 1, k, 0, 512, 128, 1, p, prior, 1,
            64, p, p,
            table, 8, wrap, 16, 100, 32, 4, 128, window, 0.1, null, 0, 0, 0,
            p, 4096, 128, null, null, null)
    # prefill: a ring table needs the run's own k/v (mixed source) and a
    # window no wider than the ring; prior context needs a block table
    for k, window in ((null, 64), (p, 0), (p, 129)):
        assert prefill(k, p, p, 8, window) == tm._lib.TMOPT_EINVAL
        assert b"ring table" in lib.tmopt_last_error()
    rc = lib.tmopt_attn_prefill_varlen(
        p, 4096, 128, p, 0, 512, 128, 1, p, 0, 512, 128, 1, p, p, 1, 64, null,
        null, null, 0, 0, 16, 0, 32, 4, 128, 0, 0.1, null, 0, 0, 0, p, 4096,
        128, null, null, null)
    assert rc == tm._lib.TMOPT_EINVAL
    assert b"prior context needs a block table" in lib.tmopt_last_error()

    # prefill, channel-major k/v (stride_tok 1, head_dim strided): they
    # need a run stride, rows holding max_seqlen tokens, both tensors in
    # the same layout, and the packed source
    def prefill_cm(run, tok, dim, v_tok, v_dim, table=None):
        return lib.tmopt_attn_prefill_varlen(
            p, 4096, 128, p, run, tok, 128 * dim, dim, p, run, v_tok,
            128 * v_dim, v_dim, p, null, 2, 64, p if table else null,
            p if table else null, table, 8 if table else 0, 0, 16,
            100 if table else 0, 32, 4, 128, 0, 0.1, null, 0, 0, 0, p, 4096,
            128, null, null, null)
    assert prefill_cm(0, 1, 64, 1, 64) == tm._lib.TMOPT_EINVAL
    assert b"need a run stride" in lib.tmopt_last_error()
    assert prefill_cm(4 * 128 * 64, 1, 64, 512, 1) == tm._lib.TMOPT_EINVAL
    assert b"both channel-major" in lib.tmopt_last_error()
    assert prefill_cm(4 * 128 * 56, 1, 56, 1, 56) == tm._lib.TMOPT_EINVAL
    assert b"hold max_seqlen_q tokens" in lib.tmopt_last_error()
    assert prefill_cm(4 * 128 * 68, 1, 68, 1, 68) == tm._lib.TMOPT_EINVAL
    assert prefill_cm(4 * 128 * 64, 1, 64, 1, 64, table=p) == \
        tm._lib.TMOPT_EUNSUPPORTED
    assert b"only as the packed source" in lib.tmopt_last_error()
    # ring decode: whole rows per work-group must cover every row
    rc = lib.tmopt_attn_decode_ring(p, p, p, p, 4, p, 10, 32, 4, 128, 40,
                                    64, 0.1, null, 0, 8, 3, 3, p, null, p,
                                    1 << 20, null)
    assert rc == tm._lib.TMOPT_EINVAL
    assert b"do not cover" in lib.tmopt_last_error()
    # table from flat rows: the table row must hold ceil(Lg / 16) pages
    rc = lib.tmopt_decode_table_from_flat(p, 100, p, 2, p, 6, p, null)
    assert rc == tm._lib.TMOPT_EINVAL
    assert b"bt_stride" in lib.tmopt_last_error()
    assert lib.tmopt_decode_table_from_flat(null, 100, null, 0, null, 0, null,
                                            null) == 0
    # kv write: misaligned strides
    rc = lib.tmopt_kv_write_slots(p, p, 3, 8, 8, 8, p, 1, 4, 128, p, p, 10,
                                  null)
    assert rc == tm._lib.TMOPT_EUNSUPPORTED
    # zero-size work is a successful no-op
    assert lib.tmopt_kv_write_slots(null, null, 0, 0, 0, 0, null, 0, 4, 128,
                                    null, null, 0, null) == 0
    # positions check: null pointers and an empty range are refused
    rc = lib.tmopt_prefill_check_positions(null, p, 8, p, null)
    assert rc == tm._lib.TMOPT_EINVAL
    assert b"null pointer" in lib.tmopt_last_error()
    rc = lib.tmopt_prefill_check_positions(p, p, 0, p, null)
    assert rc == tm._lib.TMOPT_EINVAL
    assert b"T must be positive" in lib.tmopt_last_error()


def test_python_wrapper_asserts_before_launch(tm):
    """The reference wrappers assert dtype/contiguity before launching
    (attn_swa.py:128-132); so do ours (no device needed to trip them)."""
    import torch
    q = torch.zeros((2, 32, 128), dtype=torch.float32)
    pool = torch.zeros((4, 16, 4, 128), dtype=torch.bfloat16)
    bt = torch.zeros((2, 4), dtype=torch.int32)
    ctx = torch.ones(2, dtype=torch.int32)
    with pytest.raises(AssertionError):
        tm.decode_paged(q, pool, pool, bt, ctx, 0.1)
    with pytest.raises(AssertionError):
        tm.decode_paged(q.to(torch.bfloat16), pool, pool, bt.long(), ctx, 0.1)


def test_missing_library_fails_loudly(tm, tmp_path):
    with pytest.raises(tm.TmoptLibraryMissing):
        tm._lib.load(str(tmp_path / "absent.so"))


C_CALLER = r"""
#include <stdio.h>
#include <string.h>
#include "tmopt_attn.h"

/* A C caller of the boundary, as the reference's C++ launcher would be:
   sizes a decode workspace and gets status codes back for invalid calls,
   without a GPU (validation returns before any HIP call). */
int main(void) {
  size_t ws = tmopt_attn_decode_workspace_size(64, 32, 4, 128, 0);
  int rc = tmopt_attn_prefill_varlen(
      NULL, 0, 0, NULL, 0, 0, 0, 1, NULL, 0, 0, 0, 1, NULL, NULL, 1, 16,
      NULL, NULL, NULL, 0, 0, 16, 0, 32, 4, 128, 0, 0.1f, NULL, 0, 0, 0,
      NULL, 0, 0, NULL, NULL, NULL);
  printf("%s|%zu|%d|%s\n", tmopt_version(), ws, rc, tmopt_last_error());
  return rc == TMOPT_EINVAL && ws > 0 &&
         strstr(tmopt_last_error(), "null") != NULL ? 0 : 1;
}
"""


def test_c_program_links_and_calls(tm, tmp_path):
    """The header compiles as strict C99 and a C program links against the
    built library and calls it (no Python in between)."""
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("gcc unavailable")
    src = tmp_path / "caller.c"
    src.write_text(C_CALLER)
    exe = tmp_path / "caller"
    libdir = os.path.dirname(tm._lib.LIB_PATH)
    cc = subprocess.run(
        ["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror",
         "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe),
         "-L", libdir, "-ltmopt_attn", f"-Wl,-rpath,{libdir}"],
        capture_output=True, text=True)
    assert cc.returncode == 0, cc.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True,
                         timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    version, ws, rc, msg = run.stdout.strip().split("|", 3)
    assert version == tm.version()
    assert int(ws) > 0 and int(rc) == tm._lib.TMOPT_EINVAL
