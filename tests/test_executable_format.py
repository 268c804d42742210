"""Serialized executables: the container's header, export table and ELF
payload, every corruption the verifier must catch, and loading the ELF from
the container into a private copy whose exports a command buffer records
against (no GPU needed for any of it)."""
import struct

import pytest

HDR = struct.Struct("<8sII16s24sII5Q")   # iree_mi355x_executable_header_t


def fnv1a64(b: bytes) -> int:
    h = 0xcbf29ce484222325
    for x in b:
        h = ((h ^ x) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return h


def header(data):
    (magic, fmt, libver, arch, mime, count, _r, toff, tbytes, loff, lbytes,
     csum) = HDR.unpack_from(data)
    return dict(magic=magic, fmt=fmt, libver=libver,
                arch=arch.rstrip(b"\0").decode(), mime=mime.rstrip(b"\0").decode(),
                count=count, toff=toff, tbytes=tbytes, loff=loff, lbytes=lbytes,
                csum=csum)


@pytest.fixture(scope="module")
def container(pkg):
    return pkg.serialize_executable()


def test_container_layout(pkg, container):
    h = header(container)
    assert HDR.size == 104
    assert h["magic"] == b"MI355XEX" and h["fmt"] == 1
    assert h["libver"] == pkg.EXECUTABLE_LIBRARY_VERSION
    assert h["arch"] == "gfx950" and h["mime"] == "application/x-elf"
    assert h["toff"] == HDR.size and h["loff"] == h["toff"] + h["tbytes"]
    assert h["loff"] + h["lbytes"] == len(container)
    names = container[h["toff"] + 24 * h["count"]:h["loff"]].split(b"\0")
    assert [n.decode() for n in names[:h["count"]]] == pkg.export_names()
    table = pkg.executable_library()
    for i in range(h["count"]):
        flags, lds, threads = struct.unpack_from("<3Q", container, h["toff"] + 24 * i)
        a = table.exports.attrs[i]
        assert (flags, lds, threads) == (a.flags, a.lds_bytes, a.threads)
    with open(pkg.LIB_PATH, "rb") as f:
        assert container[h["loff"]:] == f.read()
    assert fnv1a64(container[HDR.size:]) == h["csum"]
    assert pkg.verify_executable(container) == pkg.OK


def rewrite(data, **fields):
    """Change header fields (the checksum covers only what follows)."""
    h = list(HDR.unpack_from(data))
    order = ["magic", "fmt", "libver", "arch", "mime", "count", "r", "toff",
             "tbytes", "loff", "lbytes", "csum"]
    for k, v in fields.items():
        h[order.index(k)] = v
    return HDR.pack(*h) + data[HDR.size:]


def test_verifier_catches_corruption(pkg, container):
    bad = bytearray(container)
    bad[len(bad) // 2] ^= 0x40                          # payload bit flip
    assert pkg.verify_executable(bytes(bad)) == pkg.INVALID_ARGUMENT
    assert "checksum" in pkg.last_error()
    assert pkg.verify_executable(container[:100]) == pkg.INVALID_ARGUMENT
    assert pkg.verify_executable(container[:-1]) == pkg.INVALID_ARGUMENT
    assert pkg.verify_executable(rewrite(container, magic=b"MI355XEY")) == \
        pkg.INVALID_ARGUMENT
    assert pkg.verify_executable(rewrite(container, fmt=2)) == pkg.UNSUPPORTED
    assert pkg.verify_executable(rewrite(container, libver=0x48580001)) == \
        pkg.UNSUPPORTED
    assert pkg.verify_executable(rewrite(container, arch=b"gfx942")) == \
        pkg.UNSUPPORTED
    assert "gfx942" in pkg.last_error()
    h = header(container)
    assert pkg.verify_executable(rewrite(container, lbytes=h["lbytes"] - 8)) == \
        pkg.INVALID_ARGUMENT


def test_load_rejects_a_table_that_lies(pkg, container):
    """Export names are checked against the loaded library's own table."""
    h = header(container)
    data = bytearray(container)
    at = h["toff"] + 24 * h["count"]
    assert data[at:at + 10] == b"matmul_f16"
    data[at:at + 10] = b"matmul_f32"
    body = bytes(data[HDR.size:])
    data = rewrite(bytes(data[:HDR.size]) + body, csum=fnv1a64(body))
    assert pkg.verify_executable(data) == pkg.OK
    with pytest.raises(pkg.MI355XError) as e:
        pkg.LoadedExecutable(data)
    assert e.value.status == pkg.UNSUPPORTED and "names differ" in str(e.value)


def test_load_and_record_against_the_copy(pkg, container):
    """The payload loads as its own library instance; a command buffer
    records against its table and validates through its exports."""
    exe = pkg.LoadedExecutable(container)
    try:
        assert exe.export_names() == pkg.export_names()
        own = pkg.library().iree_mi355x_executable_library_query(
            pkg.EXECUTABLE_LIBRARY_VERSION, None)
        assert exe.table_ptr and exe.table_ptr != own   # a separate instance
        cb = pkg.CommandBuffer(executable=exe)
        m, n, k = 16, 4096, 4096
        cb.dispatch("matmul_f16", pkg.matmul_constants(m, n, k, k, n, n, 0),
                    [pkg.slot(0), pkg.slot(1), pkg.slot(2)]).end()
        fake = 0x10000
        table = [(fake, m * k * 2), (fake << 8, k * n * 2), (fake << 9, m * n * 2)]
        F16 = pkg.ELEM_F16
        need = pkg.plan(pkg.make_desc(F16, F16, F16, m, n, k)).workspace_bytes
        assert cb.workspace_bytes(table, 1) == (need + 255) // 256 * 256
        del cb
    finally:
        exe.release()
