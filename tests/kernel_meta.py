"""Kernel metadata of the built library's gfx950 code objects (register counts, spills, scratch), read from the
offload bundles in its .hip_fatbin section and their AMDGPU metadata notes. Host-side file parsing only."""
import struct

import msgpack

_BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _section(elf, name):
    """Bytes of ELF64 section `name`."""
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", elf, 0x3A)
    def hdr(i):
        return struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize)
    strtab = hdr(shstrndx)
    for i in range(shnum):
        h = hdr(i)
        off = strtab[4] + h[0]
        nm = elf[off:elf.index(b"\0", off)].decode()
        if nm == name:
            return elf[h[4]:h[4] + h[5]]
    return None


def _code_objects(fatbin, arch):
    """The code objects for `arch` in a concatenation of offload bundles."""
    out, pos = [], 0
    while True:
        pos = fatbin.find(_BUNDLE_MAGIC, pos)
        if pos < 0:
            return out
        n, = struct.unpack_from("<Q", fatbin, pos + 24)
        p = pos + 32
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fatbin, p)
            triple = fatbin[p + 24:p + 24 + tlen].decode()
            p += 24 + tlen
            if arch in triple:
                out.append(fatbin[pos + off:pos + off + size])
        pos = p


def _notes_metadata(co):
    """The AMDGPU metadata (msgpack, NT_AMDGPU_METADATA = 32) of one code object's .note section."""
    note = _section(co, ".note")
    p = 0
    while p < len(note):
        namesz, descsz, ntype = struct.unpack_from("<III", note, p)
        name = note[p + 12:p + 12 + namesz]
        d0 = p + 12 + ((namesz + 3) & ~3)
        if ntype == 32 and name.startswith(b"AMDGPU"):
            return msgpack.unpackb(note[d0:d0 + descsz], raw=False)
        p = d0 + ((descsz + 3) & ~3)
    return None


def kernel_metadata(lib_path, arch="gfx950"):
    """[{name, .vgpr_count, .vgpr_spill_count, .private_segment_fixed_size, ...}] for every kernel of `arch`."""
    with open(lib_path, "rb") as f:
        elf = f.read()
    fat = _section(elf, ".hip_fatbin")
    kernels = []
    for co in _code_objects(fat, arch):
        md = _notes_metadata(co)
        for k in md.get("amdhsa.kernels", []):
            k = dict(k)
            k["name"] = k.get(".name", "")
            kernels.append(k)
    return kernels
