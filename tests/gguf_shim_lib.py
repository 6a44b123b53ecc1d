"""The stand-in GGUF reader (oracle/gguf_shim.c) seen from Python: its
handle and the reference's tensor descriptor, for tests of the
ingot_gguf_* entry points. Test infrastructure only.

The shim must be loaded with RTLD_GLOBAL before libmynah_hip.so (which takes
ingot_gguf_data as a weak symbol at load time), so these tests run in a
child process."""
from __future__ import annotations

import ctypes as C


class Handle(C.Structure):
    """The shim's handle: one mapping, the data section at data_base."""
    _fields_ = [("base", C.c_void_p), ("size", C.c_uint64), ("data_base", C.c_uint64)]


class Tensor(C.Structure):
    """ingot_tensor (third_party/ingot/include/ingot/gguf.h:41-50)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("rank", C.c_uint32),
                ("ne", C.c_uint64 * 8), ("nelem", C.c_uint64), ("nbytes", C.c_uint64),
                ("offset", C.c_uint64), ("shard", C.c_uint32)]


def tensor(qtype: int, rank: int, ne, offset: int, nbytes: int) -> Tensor:
    t = Tensor()
    t.name = b"t"
    t.type = qtype
    t.rank = rank
    n = 1
    for i, v in enumerate(ne):
        t.ne[i] = v
        n *= v
    t.nelem = n
    t.nbytes = nbytes
    t.offset = offset
    return t


def load_library():
    """libmynah_hip.so with its declared signatures (after the shim)."""
    import mynah_amd
    return mynah_amd.lib
