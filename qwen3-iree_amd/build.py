"""Build recipe for the gfx950 code object and the C-ABI shim library.

  lib/q8gemv_gfx950.hsaco  hipcc --genco --offload-arch=gfx950 of csrc/q8gemv_kernels.hip
  lib/decode_gfx950.hsaco  the same for csrc/decode_kernels.hip (decode-step kernels)
  lib/prefill_gfx950.hsaco the same for csrc/prefill_kernels.hip (batched prompt ingestion)
  lib/libq8gemv.so         g++ of csrc/q8gemv_shim.cpp and hipcc of csrc/q8gemv_noalloc.hip,
                           linked against libamdhip64

Both cross-compile without a GPU.  Run as `python qwen3-iree_amd/build.py`.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

CODE_OBJECT = LIB / "q8gemv_gfx950.hsaco"
DECODE_OBJECT = LIB / "decode_gfx950.hsaco"
PREFILL_OBJECT = LIB / "prefill_gfx950.hsaco"
SHIM = LIB / "libq8gemv.so"

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    # no packed-FP32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # kernel arguments preloaded into SGPRs at dispatch, so a kernel's first
    # address does not wait for a kernarg load (the code object keeps a
    # prologue that loads them where the firmware does not preload)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "--genco",
    "--no-gpu-bundle-output",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def _hsaco(src: Path, out: Path, extra: tuple[str, ...] = ()) -> Path:
    LIB.mkdir(exist_ok=True)
    tmp = out.with_suffix(".hsaco.tmp")
    _run([str(ROCM / "bin" / "hipcc"), *HIPCC_FLAGS, *extra, f"-I{CSRC}", str(src), "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_code_object() -> Path:
    return _hsaco(CSRC / "q8gemv_kernels.hip", CODE_OBJECT)


def build_decode_object() -> Path:
    return _hsaco(CSRC / "decode_kernels.hip", DECODE_OBJECT)


def build_prefill_object() -> Path:
    # MFMA results in ordinary VGPRs rather than AGPRs: the GEMMs scale every
    # block's products with VALU FMAs, and AGPR results would first be copied
    # out (v_accvgpr_read, 4.5 per MFMA); same instructions otherwise, same bits
    return _hsaco(CSRC / "prefill_kernels.hip", PREFILL_OBJECT,
                  ("-mllvm", "-amdgpu-mfma-vgpr-form=1"))


def build_shim() -> Path:
    """libq8gemv.so: the host shim (g++) plus q8gemv_noalloc.hip (hipcc: host
    code and the device-resident scratch array of the allocation-free entry
    point, embedded as a gfx950 fat binary)."""
    import tempfile

    LIB.mkdir(exist_ok=True)
    tmp = SHIM.with_suffix(".so.tmp")
    inc = [f"-I{ROCM / 'include'}", f"-I{REPO / 'include'}", f"-I{CSRC}"]
    with tempfile.TemporaryDirectory() as td:
        shim_o = Path(td) / "q8gemv_shim.o"
        noalloc_o = Path(td) / "q8gemv_noalloc.o"
        _run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-fPIC", "-c",
              "-D__HIP_PLATFORM_AMD__", *inc, str(CSRC / "q8gemv_shim.cpp"), "-o", str(shim_o)])
        _run([str(ROCM / "bin" / "hipcc"), "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC",
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-c", *inc,
              str(CSRC / "q8gemv_noalloc.hip"), "-o", str(noalloc_o)])
        _run(["g++", "-shared", "-fPIC", str(shim_o), str(noalloc_o),
              f"-L{ROCM / 'lib'}", "-lamdhip64", "-ldl", f"-Wl,-rpath,{ROCM / 'lib'}",
              "-o", str(tmp)])
    os.replace(tmp, SHIM)
    return SHIM


# sources of each code object (the kernel file and the device headers it
# includes)
OBJECT_SOURCES = {
    "q8gemv": ("q8gemv_kernels.hip", "q8_device.h"),
    "decode": ("decode_kernels.hip", "decode_device.h", "q8_device.h"),
    "prefill": ("prefill_kernels.hip", "prefill_split.h", "decode_device.h", "q8_device.h"),
}


def source_digest(code_object: str = "q8gemv") -> str:
    """sha256 (16 hex digits) over the sources of one code object: the build
    a profile's figures belong to.  Computed from the files, so it can be
    checked where the tree has no git history."""
    import hashlib

    h = hashlib.sha256()
    for name in OBJECT_SOURCES[code_object]:
        h.update(name.encode())
        h.update((CSRC / name).read_bytes())
    return h.hexdigest()[:16]


def kernel_digest(name: str, code_object: Path = CODE_OBJECT) -> str | None:
    """sha256 (16 hex digits) of one kernel's machine code and its kernel
    descriptor (`name` and `name.kd` in the code object's ELF symbol table,
    the descriptor without its bytes 16-23: the offset to the code, which
    moves when other kernels change): the build a profile of that kernel
    belongs to, unchanged by edits to other kernels of the same sources.
    None if the kernel is absent."""
    import hashlib
    import struct

    data = Path(code_object).read_bytes()
    if data[:4] != b"\x7fELF" or data[4] != 2:
        return None
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", data, 0x3A)
    secs = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    h = hashlib.sha256()
    found = False
    for sec in secs:
        if sec[1] != 2:  # SHT_SYMTAB
            continue
        strtab = secs[sec[6]]
        for off in range(sec[4], sec[4] + sec[5], 24):
            st_name, _info, _other, shndx, value, size = struct.unpack_from("<IBBHQQ", data, off)
            end = data.index(b"\0", strtab[4] + st_name)
            sym = data[strtab[4] + st_name:end].decode()
            if sym in (name, name + ".kd") and size and shndx < len(secs):
                tgt = secs[shndx]
                start = tgt[4] + (value - tgt[3])
                body = bytearray(data[start:start + size])
                if sym.endswith(".kd") and len(body) >= 24:
                    body[16:24] = bytes(8)  # kernel_code_entry_byte_offset
                h.update(sym.encode())
                h.update(bytes(body))
                found = found or sym == name
    return h.hexdigest()[:16] if found else None


def build_all() -> tuple[Path, Path, Path, Path]:
    return build_code_object(), build_decode_object(), build_prefill_object(), build_shim()


if __name__ == "__main__":
    for path in build_all():
        print(path)
    sys.exit(0)
