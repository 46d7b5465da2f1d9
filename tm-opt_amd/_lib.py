"""ctypes binding of libtmopt_attn.so (the C ABI declared in
include/tmopt_attn.h).

The library is built in-tree by ``build.py`` into ``lib/libtmopt_attn.so``.
There is no fallback: if the library is missing every entry point raises
``TmoptLibraryMissing`` so a GPU run can never silently take another path.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libtmopt_attn.so")

TMOPT_OK = 0
TMOPT_EINVAL = -1
TMOPT_EUNSUPPORTED = -2
TMOPT_EWORKSPACE = -3
TMOPT_ELAUNCH = -4


class TmoptLibraryMissing(RuntimeError):
    """libtmopt_attn.so has not been built (run __graft_entry__.build())."""


class TmoptError(RuntimeError):
    """A C-ABI entry point returned a negative status."""

    def __init__(self, status, fn, message):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


_c_i32 = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_c_ptr = ctypes.c_void_p
_c_size = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/tmopt_attn.h one to one
SIGNATURES = {
    "tmopt_last_error": (ctypes.c_char_p, []),
    "tmopt_version": (ctypes.c_char_p, []),
    "tmopt_kv_write_slots": (_c_i32, [
        _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64,
        _c_i32, _c_i32, _c_ptr, _c_ptr, _c_i64, _c_ptr]),
    "tmopt_kv_write_paged": (_c_i32, [
        _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_ptr, _c_ptr,
        _c_i32, _c_i32, _c_ptr, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
        _c_ptr, _c_ptr, _c_i64, _c_ptr]),
    "tmopt_kv_append_rows": (_c_i32, [
        _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i32, _c_i32, _c_ptr, _c_i64,
        _c_i32, _c_i32, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_i64, _c_ptr]),
    "tmopt_attn_decode_default_workgroups": (_c_i32, [_c_i32]),
    "tmopt_attn_decode_workspace_size": (_c_size, [
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "tmopt_attn_decode_paged": (_c_i32, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i32, _c_ptr, _c_i32,
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_f32, _c_ptr,
        _c_i32, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "tmopt_attn_decode_ring": (_c_i32, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i32, _c_ptr, _c_i32, _c_i32,
        _c_i32, _c_i32, _c_i64, _c_i32, _c_f32, _c_ptr, _c_i32, _c_i32,
        _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "tmopt_decode_table_from_flat": (_c_i32, [
        _c_ptr, _c_i64, _c_ptr, _c_i32, _c_ptr, _c_i64, _c_ptr, _c_ptr]),
    "tmopt_attn_decode_paged_noalloc": (_c_i32, [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i32, _c_ptr, _c_i32,
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_f32, _c_ptr,
        _c_i32, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr]),
    "tmopt_attn_prefill_varlen": (_c_i32, [
        _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_ptr, _c_ptr, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr,
        _c_i64, _c_i32, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
        _c_f32, _c_ptr, _c_i64, _c_i64, _c_i32,
        _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr]),
    "tmopt_prefill_check_positions": (_c_i32, [
        _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_ptr]),
}

_lock = threading.Lock()
_lib = None


def load(path=None):
    """Load (once) and return the configured ctypes library."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise TmoptLibraryMissing(
                f"{p} not found: build the HIP library first "
                "(python -c 'import __graft_entry__ as g; g.build()')")
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def call(name, *args):
    """Invoke an int-returning entry point; raise TmoptError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != TMOPT_OK:
        msg = lib.tmopt_last_error().decode(errors="replace")
        raise TmoptError(rc, name, msg)
    return rc


def version():
    return load().tmopt_version().decode()
