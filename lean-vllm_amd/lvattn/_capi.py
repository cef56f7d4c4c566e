"""ctypes binding of ``liblvattn.so``: the C ABI declared in ``include/lvattn.h``.

Loading order matters: torch is imported first, so the library's ``libamdhip64.so.7`` dependency binds to the
HIP runtime torch already loaded (both carry that soname) and torch's streams and allocations are valid here.
There is no fallback: if the library is missing or fails to load, every call raises.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch  # noqa: F401  -- loads the HIP runtime this library must share

LIBRARY = Path(__file__).resolve().parent / "liblvattn.so"

# name -> (restype, argtypes), exactly the prototypes of include/lvattn.h
_P = c_void_p
_PROTOTYPES = {
    "lv_last_error": (ctypes.c_char_p, []),
    "lv_abi_version": (ctypes.c_int, []),
    "lv_pack": (ctypes.c_int, [_P, _P, _P, _P, c_int32, c_int32, c_int32, c_int32, c_int32,
                               _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int32, _P]),
    "lv_store_kvcache": (ctypes.c_int, [_P, _P, c_int64, c_int64, c_int32, c_int32, c_int32, _P, _P,
                                        c_int64, c_int64, c_int64, c_int32, _P, c_int32, _P]),
    "lv_store_latents": (ctypes.c_int, [_P, c_int64, c_int32, c_int32, _P, _P, c_int32, _P]),
    "lv_paged_attention_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                                                      c_int32]),
    "lv_paged_attention": (ctypes.c_int, [_P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int32, _P,
                                          c_int64, _P, _P, _P, c_int32, c_int32, c_int32, c_int32, c_int32,
                                          c_float, c_int32, c_int32, _P, c_int64, c_int64, _P, c_size_t,
                                          c_int32, c_int32, c_int32, c_int32, _P]),
    "lv_paged_attention_launch_info": (ctypes.c_int, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64,
                                                      c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                                                      _P]),
    "lv_paged_attention_static": (ctypes.c_int, [_P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int32,
                                                 _P, c_int64, _P, _P, _P, c_int32, c_int32, c_int32, c_int32,
                                                 c_int32, c_float, c_int32, c_int32, _P, c_int64, c_int64, c_int32,
                                                 c_int32, c_int32, c_int32, _P]),
    "lv_merge_attn_states": (ctypes.c_int, [_P, c_int64, c_int64, _P, c_int64, c_int64, _P, c_int64, c_int64,
                                            _P, c_int64, c_int64, _P, c_int64, c_int64, c_int32, c_int32,
                                            c_int32, c_int32, _P]),
    "lv_varlen_attention": (ctypes.c_int, [_P, c_int64, c_int64, _P, c_int64, c_int64, _P, c_int64, c_int64, _P, _P,
                                           c_int32, c_int32, c_int32, c_int32, c_int32, c_float, c_int32, c_int32,
                                           _P, c_int64, c_int64, _P, c_int64, c_int64, c_int32, _P]),
    "lv_varlen_context_attention": (ctypes.c_int, [_P, c_int64, c_int64, _P, c_int64, c_int64, _P, c_int64, c_int64,
                                                   _P, _P, _P, c_int64, c_int64, _P, c_int64, c_int64, _P, c_int32,
                                                   c_int32, c_int32, c_int32, c_int32, c_float, c_int32, _P, c_int64,
                                                   c_int64, _P, c_int64, c_int64, c_int32, _P]),
    "lv_mla_decode_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32]),
    "lv_mla_decode": (ctypes.c_int, [_P, c_int64, c_int64, _P, c_int64, c_int64, c_int32, _P, c_int64, _P, c_int32,
                                     c_int32, c_int32, c_int32, c_int32, c_float, c_int32, _P, c_int64, c_int64,
                                     _P, c_size_t, c_int32, _P]),
}

LV_OK, LV_EINVAL, LV_EHIP = 0, 1, 2
DTYPES = {torch.bfloat16: 0, torch.float16: 1}
# LV_KERNEL_* of lv_launch_info: the launches a paged-attention step makes
KERNELS = {0: "none", 1: "decode_list", 2: "decode_beside", 3: "decode_grid", 4: "prompt_list", 5: "prompt_overlap",
           6: "mixed_small"}


class LaunchInfo(ctypes.Structure):
    """``lv_launch_info`` of include/lvattn.h."""

    _fields_ = [(name, c_int32) for name in ("decode_kernel", "decode_workgroups", "prompt_kernel",
                                              "prompt_workgroups", "kv_heads_per_item", "two_streams",
                                              "keys_per_split", "max_splits", "splitk_merge")]

    def as_dict(self) -> dict:
        d = {name: getattr(self, name) for name, _ in self._fields_}
        d["decode_kernel"] = KERNELS[d["decode_kernel"]]
        d["prompt_kernel"] = KERNELS[d["prompt_kernel"]]
        d["two_streams"] = bool(d["two_streams"])
        d["splitk_merge"] = bool(d["splitk_merge"])
        return d


_lib: ctypes.CDLL | None = None


class LvError(RuntimeError):
    """A non-zero status from the C ABI, with the library's message."""


def library_path() -> Path:
    return LIBRARY


def load() -> ctypes.CDLL:
    """The loaded library; raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise LvError(f"{LIBRARY} is not built; run __graft_entry__.build() (or python -m lvattn._build)")
        lib = ctypes.CDLL(str(LIBRARY))
        for name, (restype, argtypes) in _PROTOTYPES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue  # reported by exported_symbols / the tests, not at load
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def exported_symbols() -> dict[str, bool]:
    lib = load()
    return {name: hasattr(lib, name) for name in _PROTOTYPES}


_fns: dict = {}


def call(name: str, *args):
    """Call ``name`` and raise ``LvError`` with the library's message on a non-zero status."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != LV_OK:
        msg = load().lv_last_error().decode(errors="replace")
        raise LvError(f"{name}: {msg} (status {rc})")
    return rc


def query(name: str, *args):
    """Call a function returning a value (no status)."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    return fn(*args)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def launch_info(*args) -> dict:
    """``lv_paged_attention_launch_info`` for the shape arguments ``args`` (as the header orders them, without the
    output struct), as a dict with kernel names."""
    info = LaunchInfo()
    call("lv_paged_attention_launch_info", *args, ctypes.byref(info))
    return info.as_dict()
