"""tm-opt paged attention, MI355X-native.

Hand-written gfx950 HIP kernels behind a C ABI (include/tmopt_attn.h,
lib/libtmopt_attn.so), reached from PyTorch-ROCm through ctypes:

  attn      native entry points: kv_write_slots / kv_write_paged /
            kv_append_rows,
            decode_paged / decode_ring (split-KV + LSE combine),
            decode_paged_noalloc, prefill_varlen (MFMA),
            prefill_check_positions.
  compat    the reference's call signatures (attn_swa, attn_global,
            attn_prefill_fused) over the native kernels.
  graph     hipGraph capture of the decode step and of the adapters with
            GraphRunner's bucket semantics (AttnGraphRunner).
  workloads seeded synthetic inputs of the benchmark configurations.

The directory name is not a Python identifier; import it with
importlib.import_module("tm-opt_amd").
"""
from . import _lib
from ._lib import TmoptError, TmoptLibraryMissing, version
from .attn import (HEAD_DIM, PAGE_SIZE, decode_default_workgroups,
                   decode_paged, decode_paged_noalloc, decode_ring,
                   decode_table_from_flat, decode_workspace,
                   decode_workspace_size, kv_append_rows,
                   kv_write_paged, kv_write_slots, prefill_check_positions,
                   prefill_varlen)
from .compat import (attn_global, attn_prefill_chunk_global,
                     attn_prefill_chunk_swa, attn_prefill_fused, attn_swa,
                     prefill_chunk_state)

__all__ = [
    "TmoptError", "TmoptLibraryMissing", "version", "HEAD_DIM", "PAGE_SIZE",
    "decode_default_workgroups", "decode_paged", "decode_paged_noalloc",
    "decode_ring", "decode_table_from_flat", "decode_workspace",
    "prefill_check_positions",
    "decode_workspace_size", "kv_append_rows", "kv_write_paged",
    "kv_write_slots",
    "prefill_varlen", "attn_swa", "attn_global", "attn_prefill_fused",
    "attn_prefill_chunk_swa", "attn_prefill_chunk_global",
    "prefill_chunk_state",
]
