"""GGUF v3 weight files on liblxops (the reference's checkpoint format,
docs/WEIGHT_FORMAT.md of Larynx): parse, list, and upload to the device.

`GgufFile(path)` parses the header (and with device=True streams the data
section into one device allocation); the model loaders are FlowDecoder.load and
Qwen2LM.load, which resolve the reference's tensor names.
"""
import ctypes as C

from ._lib import LX_GGUF_HOST_ONLY, check, lib

GGML_TYPES = {0: "F32", 1: "F16", 24: "I8", 25: "I16", 26: "I32", 27: "I64", 28: "F64",
              30: "BF16"}


class GgufFile:
    """A parsed GGUF v3 file.  device=False parses the header only (no GPU)."""

    def __init__(self, path, device=True):
        h = C.c_void_p()
        check(lib.lx_gguf_open(str(path).encode(), 0 if device else LX_GGUF_HOST_ONLY,
                               C.byref(h)))
        self._h = h
        self.device = device

    def close(self):
        if getattr(self, "_h", None):
            lib.lx_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass

    def __len__(self):
        return lib.lx_gguf_n_tensors(self._h)

    def info(self, i):
        """(name, ggml type, torch shape, nbytes) of tensor i."""
        name, typ, nd = C.c_char_p(), C.c_int(), C.c_int()
        ne = (C.c_int64 * 4)()
        nb = C.c_uint64()
        check(lib.lx_gguf_tensor_info(self._h, i, C.byref(name), C.byref(typ), C.byref(nd), ne,
                                      C.byref(nb)))
        shape = tuple(int(ne[d]) for d in range(nd.value))[::-1]
        return name.value.decode(), typ.value, shape, nb.value

    def tensors(self):
        return [self.info(i) for i in range(len(self))]

    def find(self, name):
        return lib.lx_gguf_find(self._h, name.encode())

    def data_ptr(self, name):
        """Device pointer of a tensor (None when parsed host-only or absent)."""
        i = self.find(name)
        return None if i < 0 else lib.lx_gguf_tensor_data(self._h, i)

    def metadata(self, key):
        v = lib.lx_gguf_get_string(self._h, key.encode())
        return None if v is None else v.decode()
