"""CPU tests of the GEMM device-program ABI (include/hk.h, hk_module_* / hk_launch_kernel_with_args):
the argument structs keep the reference's layout, the built code object is a gfx950 ELF that
defines the reference's 18 program names, and the loader's image checks reject what the reference's
artifact reader rejects (deepgemm/artifact.rs:18-22) before any device work."""
import ctypes
import os
import struct

import pytest

from rust_ascend_hip import _lib
from rust_ascend_hip._lib import HkEpilogue, HkGm

PROGRAM_NAMES = sorted(
    [f"ruda_rust_bf16_{kind}_{ta}{tb}_{out}" for kind in ("dense", "batched") for ta in "nt" for tb in "nt"
     for out in ("bf16", "f32")] + [f"ruda_rust_bf16_mgrouped_nt_{out}" for out in ("bf16", "f32")])


def test_argument_structs_match_the_reference_layout():
    """deepgemm/native.rs:96: GmPtr 24 bytes (stride_outer at 8), Epilogue 32 bytes (sfd at 8, n at 24)."""
    assert len(PROGRAM_NAMES) == 18
    assert ctypes.sizeof(HkGm) == 24 and ctypes.alignment(HkGm) == 8 and HkGm.stride_outer.offset == 8
    assert HkGm.stride_batch.offset == 16
    assert ctypes.sizeof(HkEpilogue) == 32 and HkEpilogue.sfd.offset == 8 and HkEpilogue.stride.offset == 16
    assert HkEpilogue.n.offset == 24 and HkEpilogue.pad1.offset == 28


def _image():
    if not os.path.exists(_lib.PROGRAMS_PATH):
        pytest.fail(f"{_lib.PROGRAMS_PATH} is missing: build with __graft_entry__.build()")
    with open(_lib.PROGRAMS_PATH, "rb") as f:
        return f.read()


def _elf_functions(data):
    """Names of the STT_FUNC symbols of a little-endian ELF64 image."""
    shoff, = struct.unpack_from("<Q", data, 40)
    shentsize, shnum = struct.unpack_from("<HH", data, 58)
    sections = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    names = set()
    for _, sh_type, _, _, off, size, link, _, _, entsize in sections:
        if sh_type not in (2, 11):  # SHT_SYMTAB, SHT_DYNSYM
            continue
        str_off = sections[link][4]
        for j in range(size // entsize):
            st_name, st_info = struct.unpack_from("<IB", data, off + j * entsize)
            if st_info & 0xF == 2:  # STT_FUNC
                end = data.index(b"\0", str_off + st_name)
                names.add(data[str_off + st_name:end].decode())
    return names


def test_code_object_is_gfx950_and_defines_every_program():
    data = _image()
    assert data[:6] == b"\x7fELF\x02\x01"
    e_type, e_machine = struct.unpack_from("<HH", data, 16)
    e_flags, = struct.unpack_from("<I", data, 48)
    assert (e_type, e_machine) == (3, 224)  # ET_DYN, EM_AMDGPU
    assert e_flags & 0xFF == 0x4F  # EF_AMDGPU_MACH_AMDGCN_GFX950
    assert set(PROGRAM_NAMES) <= _elf_functions(data)


def _load(image, size=None):
    lib = _lib.load()
    buf = ctypes.create_string_buffer(image, len(image))
    out = ctypes.c_void_p(123)
    st = lib.hk_module_load_data(None, buf, len(image) if size is None else size, ctypes.byref(out))
    assert out.value is None  # cleared on every failure
    return st, _lib.last_error()


def test_loader_rejects_bad_images_before_the_context():
    data = _image()
    assert _load(b"\0" * 32) == (_lib.LOAD_ERROR, "invalid code object size 32")
    st, msg = _load(b"__CLANG_OFFLOAD_BUNDLE__" + data[24:])
    assert st == _lib.LOAD_ERROR and "unbundled" in msg
    wrong_machine = bytearray(data)
    wrong_machine[18:20] = struct.pack("<H", 62)  # EM_X86_64
    st, msg = _load(bytes(wrong_machine))
    assert st == _lib.LOAD_ERROR and "not an AMDGPU code object" in msg
    gfx942 = bytearray(data)
    gfx942[48] = 0x4C  # EF_AMDGPU_MACH_AMDGCN_GFX942
    st, msg = _load(bytes(gfx942))
    assert st == _lib.LOAD_ERROR and "another GPU" in msg
    st, msg = _load(data[:len(data) // 2])
    assert st == _lib.LOAD_ERROR and "truncated" in msg
    # a valid image reaches the context check
    st, msg = _load(data)
    assert st == _lib.NOT_INITIALIZED, msg


def test_program_entry_points_need_a_context():
    lib = _lib.load()
    fn = ctypes.c_void_p()
    assert lib.hk_module_get_function(None, None, b"ruda_rust_bf16_dense_nt_bf16", ctypes.byref(fn)) == \
        _lib.NOT_INITIALIZED
    argv = (ctypes.c_void_p * 9)()
    assert lib.hk_launch_kernel_with_args(None, None, 32, argv) == _lib.NOT_INITIALIZED
    assert lib.hk_module_unload(None, ctypes.c_void_p(8)) == _lib.NOT_INITIALIZED
    assert lib.hk_module_unload(None, None) == _lib.OK  # like free(NULL)
    out = ctypes.c_void_p()
    assert lib.hk_group_ends_data(None, None, ctypes.byref(out)) == _lib.NOT_INITIALIZED
