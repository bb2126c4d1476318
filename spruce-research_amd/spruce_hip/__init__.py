"""ctypes binding of libspruce_hip.so, the gfx950 kernels of the sparse-prefill path.

The library exports a plain C ABI (``include/spruce_hip.h``): device pointers,
int64 element strides and a ``hipStream_t``.  This module only marshals torch
tensors into those arguments; it never computes anything itself.  If the
library has not been built the calls raise ``RuntimeError`` -- there is no
CPU fallback.

torch is imported before the library is opened so that the library binds to
the HIP runtime torch already loaded (both carry the SONAME
``libamdhip64.so.7``), keeping one runtime and one set of streams per process.
"""
import ctypes
import json
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libspruce_hip.so")

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

KERNEL_VARIANTS = (
    "single_head",
    "single_head_causal",
    "single_head_prescale",
    "single_head_qtile",
    "tiled_gqa",
)

_i64 = ctypes.c_int64
_p = ctypes.c_void_p
_STRIDES = ctypes.POINTER(_i64)

# name -> argument types, mirroring include/spruce_hip.h.
_SIGNATURES = {
    "spruce_last_error": [ctypes.c_char_p, ctypes.c_size_t],
    "spruce_kernel_metadata": [ctypes.c_int, _i64, _i64, _i64, ctypes.c_char_p, ctypes.c_size_t],
    "spruce_sparse_prefill_index": [
        _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _i64,
        _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
        _p, _STRIDES, _p],
    "spruce_causal_prefill": [
        _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
        ctypes.c_int, _p, _STRIDES, _p, _p, _i64, _p],
    "spruce_sparse_prefill_csr": [
        _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _p, _p, _i64, _p,
        _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
        _p, _STRIDES, _p],
    "spruce_selector_pool": [
        _p, _STRIDES, _p, _STRIDES, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _p, _p],
    "spruce_gate_project": [_p, _p, _i64, _i64, _i64, _p, _p],
    "spruce_gate_project2": [_p, _p, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _p],
    "spruce_gate_project_levels": [ctypes.POINTER(_p), _STRIDES, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _i64,
                                   _p, ctypes.c_int, _p],
    "spruce_gate_scores": [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, _p, _p],
    "spruce_causal_topk": [_p, _i64, _i64, _i64, _i64, _p, _p],
    "spruce_select_flat_supported": [_i64, _i64, _i64, _i64, ctypes.c_int, _i64],
    "spruce_selector_pool_project": [
        _p, _STRIDES, _p, _STRIDES, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _p, _i64, _p, _p, _p],
    "spruce_select_flat": [
        _p, _STRIDES, _p, _STRIDES, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _p, _i64, ctypes.c_float,
        _i64, _p, _i64, _p, _p],
    "spruce_teacher_block_mass": [
        _p, _STRIDES, _p, _STRIDES, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int,
        _p, _p, ctypes.c_size_t, _p],
    "spruce_teacher_block_mass_schedule": [
        _p, _STRIDES, _p, _STRIDES, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int,
        _p, _p, ctypes.c_size_t, ctypes.c_int, _p],
    "spruce_teacher_schedule": [_i64, _i64, _i64, _i64, _i64, ctypes.c_size_t],
    "spruce_teacher_targets": [
        _p, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p, _p, _p, _p],
    "spruce_teacher_group_mass": [_p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p],
    "spruce_pack_selected_ids": [_p, ctypes.c_int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "spruce_pack_selected_mask": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "spruce_proto_pool": [_p, _STRIDES, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _p],
    "spruce_proto_pool_qk": [_p, _STRIDES, _p, _STRIDES, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int,
                             _p, _p, _p],
    "spruce_kv_summary": [
        _p, _STRIDES, _p, _STRIDES, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _p, _p, _i64,
        _p, _p, _p, _p, _p, ctypes.c_size_t, _p],
    "spruce_kv_summary_noalloc": [
        _p, _STRIDES, _p, _STRIDES, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _p, _p, _i64,
        _p, _p, _p, _p, _p],
    "spruce_group_avg_tokens": [_p, _STRIDES, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _p],
    "spruce_sparse_prefill_index_summaries": [
        _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _i64,
        _p, _STRIDES, _i64, _p, _p, _p, ctypes.c_int, _i64, _i64,
        _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
        _p, _STRIDES, _p],
    "spruce_sparse_prefill_index_amask": [
        _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _i64, _p, _STRIDES, _i64, _i64, _i64,
        ctypes.c_int, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
        _p, _STRIDES, _p],
    "spruce_sparse_prefill_index_masked": [
        _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _i64, _p, _i64,
        _p, _STRIDES, _i64, _p, _p, _p, ctypes.c_int, _i64, _i64,
        _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
        _p, _STRIDES, _p],
    "spruce_residual_frontier": [_p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _p],
    "spruce_tree_merge_level": [_p, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _p],
    "spruce_tree_merge_levels": [_p, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _p, _i64, _p],
    "spruce_tree_traverse": [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p, _i64,
                             ctypes.c_int, _p],
    "spruce_gate_candidate_scores": [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p, _p],
    "spruce_sparse_prefill_mask": [
        _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _p, _STRIDES, _i64,
        _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
        _p, _STRIDES, _p],
}

SIZE_MAX = ctypes.c_size_t(-1).value

_lib = None


def is_built():
    return os.path.exists(LIB_PATH)


def lib():
    """Open libspruce_hip.so once; raise RuntimeError if it is missing."""
    global _lib
    if _lib is None:
        if not is_built():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() "
                "(make -C spruce-research_amd/csrc)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        handle.spruce_version.restype = ctypes.c_char_p
        handle.spruce_version.argtypes = []
        for name in ("spruce_teacher_workspace_bytes", "spruce_teacher_workspace_bytes_min"):
            getattr(handle, name).restype = ctypes.c_size_t
            getattr(handle, name).argtypes = [_i64, _i64, _i64]
        handle.spruce_teacher_schedule_workspace_bytes.restype = ctypes.c_size_t
        handle.spruce_teacher_schedule_workspace_bytes.argtypes = [_i64, _i64, _i64, ctypes.c_int]
        handle.spruce_kv_summary_workspace_bytes.restype = ctypes.c_size_t
        handle.spruce_kv_summary_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64]
        handle.spruce_select_flat_workspace_bytes.restype = _i64
        handle.spruce_select_flat_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64]
        _lib = handle
    return _lib


def last_error():
    buf = ctypes.create_string_buffer(1024)
    lib().spruce_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc, what):
    """Map an ABI return code to the reference's exception types."""
    if rc == 0:
        return
    message = last_error()
    if rc < 0:
        raise ValueError(message)
    raise RuntimeError(f"{what} failed with hipError {rc}: {message}")


def strides(t, order=None):
    """int64[4] element strides of a 4-D tensor (optionally permuted)."""
    s = t.stride() if order is None else tuple(t.stride(i) for i in order)
    if len(s) != 4:
        raise ValueError(f"expected a 4-D tensor, got {t.dim()}-D")
    return (_i64 * 4)(*s)


def strides5(t):
    """int64[5] element strides of a 5-D tensor."""
    if t.dim() != 5:
        raise ValueError(f"expected a 5-D tensor, got {t.dim()}-D")
    return (_i64 * 5)(*t.stride())


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def dtype_code(t):
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; expected bfloat16, float16 or float32")


def variant_code(kernel_variant):
    if kernel_variant not in KERNEL_VARIANTS:
        raise ValueError(
            f"kernel_variant must be one of {KERNEL_VARIANTS}, got {kernel_variant!r}")
    return KERNEL_VARIANTS.index(kernel_variant)


def launch_config(kernel_variant, Hq, Hkv, D):
    """The launch configuration the library uses for a shape (parsed JSON)."""
    buf = ctypes.create_string_buffer(1024)
    check(lib().spruce_kernel_metadata(variant_code(kernel_variant), Hq, Hkv, D, buf, len(buf)),
          "spruce_kernel_metadata")
    return json.loads(buf.value.decode())


def version():
    return lib().spruce_version().decode()
