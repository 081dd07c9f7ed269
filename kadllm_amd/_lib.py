"""ctypes binding of libkadllm_hip.so (the C ABI declared in include/kadllm_hip.h).

The library is built in-tree by ``kadllm_amd.csrc.build``.  torch is imported
first so that the library binds to the HIP runtime torch already loaded (both
carry the SONAME libamdhip64.so.7), giving one runtime, one set of streams and
one device allocator per process.  There is no fallback: if the library is
missing or fails to load, every operator raises.
"""

import ctypes
import os
import re

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkadllm_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                           "include", "kadllm_hip.h")

KAD_OK = 0
ERRORS = {-1: "invalid argument", -2: "unsupported", -3: "HIP error"}
DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_P, _L, _I, _F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
_CTYPES = {"p": _P, "l": _L, "i": _I, "f": _F, "s": _P}

# argument signatures, one letter per parameter (p pointer, l int64, i int,
# f float, s stream), in the order of include/kadllm_hip.h
SIGNATURES = {
    "kad_gdn_suffix_replay": "ppplli" "pipil" "pi" "pl" "iiiiiii" "f" "s",
    "kad_gdn_suffix_replay_conv": "pl" "plllip" "pipil" "pi" "pl" "iiiiiii" "f" "s",
    "kad_gdn_suffix_replay_conv_gated": "pl" "plllip" "pipil" "pi" "plpfi" "pl" "iiiiiii" "f"
                                        "s",
    "kad_gdn_suffix_replay_conv_gated_parents": "plpipl" "plllip" "pipil" "pi" "plpf" "pl"
                                                "iiiiiii" "f" "s",
    "kad_causal_conv_suffix": "plll" "pllli" "pip" "plll" "iiiiii" "s",
    "kad_gemm_bf16": "plplplpl" "iiii" "s",
    "kad_gemm_bf16_tiled": "plplplpl" "iiiii" "s",
    "kad_gemm_bf16_conv_workspace_bytes": "iip",
    "kad_gemm_bf16_conv": "plplpl" "iiii" "pip" "pl" "s",
    "kad_rmsnorm": "plpfpllifs",
    "kad_rmsnorm_gated": "plplpplliifs",
    "kad_gdn_gates": "plplpppplis",
    "kad_qk_norm_rope": "plli" "pp" "lllll" "ii" "p" "ll" "f" "i" "s",
    "kad_scatter_heads": "pliipllllls",
    "kad_embedding": "ppplils",
    "kad_prefix_attention_decode": "plll" "pplll" "plll" "plll" "pp" "lll" "plll" "iiiiiii" "f" "s",
    "kad_prefix_attention_decode_ex": "plll" "pplll" "plll" "plll" "pp" "lll" "plll" "iiiiiiii" "f"
                                      "s",
    "kad_attention_prefill": "plll" "pplll" "plll" "plll" "iiiii" "f" "s",
    "kad_beam_row_select": "pilplpiiiipps",
    "kad_beam_select_noalloc": "pilplpiiiipppps",
    "kad_gdn_recurrent": "ppplli" "pipil" "pii" "plp" "iiiiiif" "s",
    "kad_attention_general": "plll" "pplll" "plll" "plll" "pp" "lll" "plll" "iiiiiiiii" "f" "s",
    "kad_beam_merge_select": "ppiiiipppps",
    "kad_beam_merge_select_wide_workspace_bytes": "iip",
    "kad_beam_merge_select_wide": "ppiiiippppp" "l" "s",
    "kad_beam_history": "piipppiis",
    "kad_gather_beam_rows": "pli" "pli" "i" "l" "p" "iii" "s",
    "kad_gdn_chunk_workspace_bytes": "iiiip",
    "kad_gdn_chunk": "ppplli" "pipil" "pii" "plp" "pl" "iiiiii" "fi" "s",
    "kad_gdn_chunk_gated": "ppplli" "pipil" "pii" "plp" "pl" "iiiiii" "f" "plpf" "s",
    "kad_causal_conv_prefill": "plpplpiiiis",
    "kad_gemm_f32": "plplplpl" "iiii" "s",
    "kad_rmsnorm_f32": "plpfpllifs",
    "kad_rmsnorm_gated_f32": "plplpplliifs",
    "kad_gdn_gates_f32": "plplpppplis",
    "kad_qk_norm_rope_f32": "plli" "pp" "lllll" "ii" "p" "ll" "f" "i" "s",
    "kad_embedding_f32": "ppplils",
    "kad_hbm_probe": "pplis",
    "kad_cache_prefetch": "plpls",
    "kad_selftest_mfma_f32": "ppps",
    "kad_selftest_mfma16": "ppps",
    "kad_selftest_mfma32": "ppps",
}

_lib = None


class KadLibraryError(RuntimeError):
    """Raised when the HIP library is missing or an entry point fails."""


def header_symbols():
    """Entry points declared in include/kadllm_hip.h."""
    with open(HEADER_PATH) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int)\s+(kad_\w+)\s*\(", text, re.M)))


def load():
    """Load the library (once) and declare argument types."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise KadLibraryError(
            f"{LIB_PATH} is not built; run `python -m kadllm_amd.csrc.build` "
            "(kadllm_amd has no non-HIP implementation)")
    lib = ctypes.CDLL(LIB_PATH)
    lib.kad_last_error.restype = ctypes.c_char_p
    lib.kad_last_error.argtypes = []
    lib.kad_abi_version.restype = ctypes.c_int
    lib.kad_abi_version.argtypes = []
    for name, sig in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [_CTYPES[c] for c in sig]
    _lib = lib
    return lib


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t):
    """Raw hipStream_t of torch's current stream on ``t``'s device (an int,
    which ctypes passes for the c_void_p argument)."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


_call_hook = None


def set_call_hook(hook):
    """Install (or clear with None) ``hook(name, args, launch)``, which every
    call makes instead of invoking entry point ``name`` directly; the hook
    must call ``launch()`` once (e.g. between two HIP events, for per-kernel
    timing)."""
    global _call_hook
    _call_hook = hook


def _invoke(lib, name, args):
    rc = getattr(lib, name)(*args)
    if rc != KAD_OK:
        msg = lib.kad_last_error().decode(errors="replace")
        raise KadLibraryError(f"{name} failed ({ERRORS.get(rc, rc)}): {msg}")


def call(name, *args):
    """Invoke entry point ``name``; raise KadLibraryError on a nonzero code."""
    lib = load()
    if _call_hook is None:
        _invoke(lib, name, args)
    else:
        _call_hook(name, args, lambda: _invoke(lib, name, args))


def gdn_chunk_workspace(N, T, HV, K, device):
    """A uint8 device buffer sized for kad_gdn_chunk."""
    n = ctypes.c_int64(0)
    call("kad_gdn_chunk_workspace_bytes", N, T, HV, K, ctypes.byref(n))
    return torch.empty(n.value, dtype=torch.uint8, device=device)


def dtype_code(dtype):
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None


def ptr(t):
    """Device address of a tensor (None for a null pointer); ctypes converts
    the int for the c_void_p argument."""
    return t.data_ptr() if t is not None else None


def ptr_at(address):
    """A raw device address (e.g. a column offset inside a row-strided buffer)."""
    return address
