"""ctypes bindings of libmetal_linalg.so, generated from its C headers.

The headers under include/metal_linalg/ (c_api.h: the reference's C ABI;
hip_ext.h: this build's HIP extensions) are the one description of the
library's interface.  At import they are read, every ``metal_linalg_*``
prototype becomes a ctypes function under its name without the prefix
(``metal_linalg_qr`` -> ``qr``), and every policy ``typedef struct`` becomes
a ctypes Structure with the header's field order, so a change of the C
interface needs no second edit here.

Loading needs no GPU (the device is opened at the first decomposition), so
symbol checks run anywhere.  Calls are serialised by ``lock``: the library's
device workspaces are shared by every call in the process (the reference's
PyTorch binding takes one lock for the same reason,
python-torch/metal_linalg_torch/_lib.py:24).
"""

from __future__ import annotations

import ctypes
import os
import re
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.environ.get("METAL_LINALG_LIBRARY") or os.path.join(HERE, "libmetal_linalg.so")
INCLUDE = os.environ.get("METAL_LINALG_INCLUDE") or os.path.join(os.path.dirname(HERE), "include", "metal_linalg")
HEADERS = ("c_api.h", "hip_ext.h")

if not os.path.exists(PATH):
    raise ImportError(f"metal_linalg_amd: {PATH} is not built; run `python -m metal_linalg_amd.build` "
                      f"(or __graft_entry__.build()) first")

# torch ships its own libamdhip64.so.7 under the same soname as ROCm's.  One
# process must hold one HIP runtime, or device pointers from torch are
# unknown to the library's: when torch is installed it is loaded first, so
# that the library binds to the runtime torch already uses.
try:
    import torch  # noqa: F401
except ImportError:
    pass

lib = ctypes.CDLL(PATH)
lock = threading.RLock()

OK, INVALID_ARGUMENT, RUNTIME_ERROR, OUT_OF_MEMORY = 0, 1, 2, 3
NO_LIMIT = 0xFFFFFFFF
QR_MODES = {"reduced": 0, "r": 1, "complete": 2}
# policy fields that describe the device: read back, never written
INFORMATIONAL = frozenset({"gpu_cores", "concurrent_matrices"})

# ---- the header reader ----

_SCALARS = {
    "void": None, "int": ctypes.c_int, "uint32_t": ctypes.c_uint32, "uint64_t": ctypes.c_uint64,
    "float": ctypes.c_float, "double": ctypes.c_double, "long long": ctypes.c_longlong,
    # enums pass as int
    "metal_linalg_status": ctypes.c_int, "metal_linalg_qr_mode": ctypes.c_int,
}


def _strip_comments(text: str) -> str:
    """Comments and preprocessor lines removed."""
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return "\n".join(line for line in text.splitlines() if not line.lstrip().startswith("#"))


def _ctype(decl: str, structs: dict):
    """ctypes type of a C type as written in a prototype (names dropped)."""
    decl = " ".join(decl.replace("const", " ").split())
    pointer = decl.endswith("*")
    base = decl.rstrip("* ").strip()
    if pointer:
        if base == "char":
            return ctypes.c_char_p
        if base in structs:
            return ctypes.POINTER(structs[base])
        return ctypes.c_void_p        # buffers: host or device addresses
    if base in structs:
        return structs[base]
    if base not in _SCALARS:
        raise TypeError(f"metal_linalg_amd: no ctypes mapping for C type {decl!r}")
    return _SCALARS[base]


def _split_param(param: str) -> str:
    """The type part of 'const float* a' (drop the trailing name)."""
    param = param.strip()
    if param in ("", "void"):
        return ""
    m = re.match(r"^(.*?[\s\*])(\w+)$", param)
    return m.group(1) if m else param


def _read_headers():
    text = ""
    for h in HEADERS:
        with open(os.path.join(INCLUDE, h)) as f:
            text += _strip_comments(f.read()) + "\n"
    structs = {}
    for name, body in re.findall(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*\1\s*;", text, flags=re.S):
        fields = re.findall(r"uint32_t\s+(\w+)\s*;", body)
        structs[name] = type(name, (ctypes.Structure,), {"_fields_": [(f, ctypes.c_uint32) for f in fields]})
    protos = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w\s\*]*?)\s*\b(metal_linalg_\w+)\s*\(([^()]*)\)\s*;", text):
        types = [_split_param(p) for p in params.split(",")]
        protos[name] = (_ctype(ret, structs), [_ctype(t, structs) for t in types if t])
    return structs, protos


STRUCTS, PROTOTYPES = _read_headers()


def _bind(cname: str):
    restype, argtypes = PROTOTYPES[cname]
    f = getattr(lib, cname)
    f.restype = restype
    f.argtypes = argtypes
    return f


for _cname in PROTOTYPES:
    globals()[_cname[len("metal_linalg_"):]] = _bind(_cname)
del _cname


# ---- policies ----

def policy_struct(what: str):
    """The ctypes Structure of metal_linalg_<what>_policy."""
    return STRUCTS[f"metal_linalg_{what}_policy"]


def get_policy(what: str) -> dict:
    """The routing policy of one decomposition as {field: value}."""
    read = globals()[f"{what}_policy_get"]
    with lock:
        raw = read()
    return {name: int(getattr(raw, name)) for name, _ in raw._fields_}


def set_policy(what: str, values: dict) -> None:
    """Overrides some fields of a policy; the informational ones are kept."""
    struct = policy_struct(what)
    names = [name for name, _ in struct._fields_]
    unknown = sorted(set(values) - set(names))
    if unknown:
        raise TypeError(f"unknown {what} policy field(s): {', '.join(unknown)}")
    with lock:
        merged = get_policy(what)
        merged.update({k: int(v) for k, v in values.items() if k not in INFORMATIONAL})
        globals()[f"{what}_policy_set"](ctypes.byref(struct(**merged)))


# ---- measurement helpers (hip_ext.h) ----

def kernel_time(name: str):
    """(launches, total_ms) of a timed kernel since the last reset."""
    n = ctypes.c_uint64()
    ms = ctypes.c_double()
    hip_kernel_time(name.encode(), ctypes.byref(n), ctypes.byref(ms))  # noqa: F821 (bound from the header)
    return int(n.value), float(ms.value)


def kernel_names():
    return [x for x in hip_kernel_names().decode().split("\n") if x]  # noqa: F821
