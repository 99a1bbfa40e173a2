"""A read-only GGUF (v2 / v3) table reader: metadata and tensor descriptors, so that a PTQ1_0 tensor can be streamed
to the device by name (the role of Kindi's gguf.GGUF, gguf.py, for the linear-layer weights). Nothing in the file
is executed: values are parsed by their declared types only."""
import struct

PTQ1_0, F32, BF16 = 143, 0, 30
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class GGUF(object):
    """kv: metadata dict; tensors: {name: (dims [ne0, ne1, ...], type, absolute byte offset of the data)}"""

    def __init__(self, path):
        self.path = path
        with open(path, "rb") as f:
            self._f = f
            if f.read(4) != b"GGUF":
                raise ValueError("%s: not a GGUF file" % path)
            self.version, = self._u("<I")
            if self.version not in (2, 3):
                raise ValueError("%s: GGUF version %d is not read" % (path, self.version))
            nt, nkv = self._u("<QQ")
            self.kv = {}
            for _ in range(nkv):
                key = self._str()
                self.kv[key] = self._val(self._u("<I")[0])
            infos = []
            for _ in range(nt):
                name = self._str()
                nd, = self._u("<I")
                dims = list(self._u("<%dQ" % nd))
                ty, off = self._u("<IQ")
                infos.append((name, dims, ty, off))
            align = int(self.kv.get("general.alignment", 32))
            pos = f.tell()
            self.data_start = (pos + align - 1) // align * align
        self.tensors = {n: (d, t, self.data_start + o) for n, d, t, o in infos}
        del self._f

    def _u(self, fmt):
        n = struct.calcsize(fmt)
        b = self._f.read(n)
        if len(b) != n:
            raise ValueError("%s: truncated" % self.path)
        return struct.unpack(fmt, b)

    def _str(self):
        n, = self._u("<Q")
        return self._f.read(n).decode("utf-8")

    def _val(self, ty):
        if ty in _SCALAR:
            return self._u(_SCALAR[ty])[0]
        if ty == 8:
            return self._str()
        if ty == 9:
            et, n = self._u("<IQ")
            return [self._val(et) for _ in range(n)]
        raise ValueError("%s: unknown metadata type %d" % (self.path, ty))


def load_ternary(path, name, device="cuda", W=None, chunk_rows=8192, g=None):
    """the PTQ1_0 tensor `name` of a GGUF file as a kt2 TernaryMatrix (R = the product of the outer dims, C = ne0)"""
    from .linear import load_ptq1
    g = g or GGUF(path)
    dims, ty, off = g.tensors[name]
    if ty != PTQ1_0:
        raise ValueError("%s: type %d is not PTQ1_0" % (name, ty))
    R = 1
    for x in dims[1:]:
        R *= x
    return load_ptq1(path, off, R, dims[0], device=device, W=W, chunk_rows=chunk_rows)
