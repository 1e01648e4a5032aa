"""Build the gfx950 kernel libraries and their repo-local kernel pack.

Outputs (all under ``radeon-kernels_amd/packs/gfx950``):

* ``lib/librk_pa_gfx950.so`` -- paged-attention decode C-ABI library (``include/rk_paged_attention.h``).
* ``lib/rk_pa_gfx950.so``    -- its PyTorch-ROCm binding (module ``rk_pa_gfx950``).
* ``lib/librk_kv_gfx950.so`` -- paged KV-cache C-ABI library (``include/rk_kv_cache.h``).
* ``lib/rk_kv_append_gfx950.so``, ``lib/rk_kv_copy_gfx950.so`` -- its PyTorch-ROCm bindings, one
  module per operator (a pack names one artifact file per operator), built from one source.
* ``lib/librk_sdpa_gfx950.so`` -- self-attention (prefill) C-ABI library (``include/rk_sdpa.h``).
* ``lib/rk_sdpa_gfx950.so`` -- its PyTorch-ROCm binding (module ``rk_sdpa_gfx950``).
* ``manifest.json``          -- the kernel-pack manifest (same fields as the reference's
  ``schemas/kernel-pack.schema.json``), stamped with the bindings' SHA-256 and this environment.

Each HIP source is compiled once and linked into both its C-ABI library and its bindings, so a
binding depends on no other file of the pack and the digest a dispatch entry pins covers the
kernels the binding runs.  The build also rewrites the winners' ``sha256`` and ``environment`` in
``radeon_kernels/dispatch/<operator>-1.0.json`` from ``dispatch_plan.py``.  The reference binds every
dispatch entry to the exact artifact digest and to the exact torch/Python/ROCm ABI
(src/radeon_kernels/runtime/compatibility.py:94-102), so both files are
generated after each build rather than written by hand.

Run as ``python radeon-kernels_amd/build.py`` or through ``__graft_entry__.build()``.
"""

from __future__ import annotations

import hashlib
import json
import os
import subprocess
import sys
import sysconfig
import tempfile
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_ROOT.parent
CSRC = PACKAGE_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
PACK_DIR = PACKAGE_ROOT / "packs" / "gfx950"
LIB_DIR = PACK_DIR / "lib"
CABI_NAME = "librk_pa_gfx950.so"
EXTENSION_NAME = "rk_pa_gfx950"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-FP32 VALU ops stay disabled: all fp32 math uses the scalar VALU forms.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # Every atomic in these kernels is issued by a single lane.  The atomic optimizer would rewrite
    # each into its lane-combining form, which reads the result back at once (a full memory-counter
    # wait) instead of where it is used.
    "-mllvm",
    "-amdgpu-atomic-optimizer-strategy=None",
    f"-ffile-prefix-map={REPO_ROOT}=.",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    return str(candidate) if candidate.exists() else "hipcc"


def _torch_paths() -> tuple[list[str], list[str]]:
    from torch.utils import cpp_extension

    try:
        includes = list(cpp_extension.include_paths(device_type="cuda"))
        libraries = list(cpp_extension.library_paths(device_type="cuda"))
    except TypeError:  # older torch: boolean ``cuda`` argument
        includes = list(cpp_extension.include_paths(True))
        libraries = list(cpp_extension.library_paths(True))
    rocm_include = str(Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "include")
    if rocm_include not in includes:
        includes.append(rocm_include)
    return includes, libraries


def _run(command: list[str], verbose: bool) -> subprocess.Popen:
    if verbose:
        print("+", " ".join(command), flush=True)
    return subprocess.Popen(command, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _finish(process: subprocess.Popen, what: str) -> None:
    output, _ = process.communicate()
    if process.returncode != 0:
        raise RuntimeError(f"{what} failed (exit {process.returncode}):\n{output}")


def _atomic_write(path: Path, text: str) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    handle, temporary = tempfile.mkstemp(dir=path.parent, prefix=f".{path.name}.")
    with os.fdopen(handle, "w", encoding="utf-8") as stream:
        stream.write(text)
    os.chmod(temporary, 0o644)
    os.replace(temporary, path)


def sha256_file(path: Path) -> str:
    digest = hashlib.sha256()
    with path.open("rb") as stream:
        for chunk in iter(lambda: stream.read(1 << 20), b""):
            digest.update(chunk)
    return digest.hexdigest()


class Library:
    """One HIP source compiled once (hipcc -c) and linked twice: into the C-ABI kernel library
    (hipcc -shared) and into each torch binding module (g++), so that every binding is
    self-contained -- a pack then consists of its manifest, its signature and the artifacts the
    manifest names, the release layout the reference's installer accepts (installer.py:187-220),
    and an artifact's digest covers the kernels it runs.

    ``bindings`` maps each binding module name to the operators whose dispatch entries name it; a
    pack needs one artifact file per operator, so operators sharing a source get one module each,
    all built from the same binding source."""

    def __init__(self, hip_source: str, cabi_name: str, binding_source: str,
                 bindings: dict[str, tuple[str, ...]], units: tuple[tuple[str, tuple[str, ...]], ...] = (),
                 unit_flags: tuple[str, ...] = ()) -> None:
        self.hip_source = CSRC / hip_source
        self.cabi_name = cabi_name
        self.binding_source = CSRC / binding_source
        self.bindings = bindings
        # Further HIP compilations linked into the same library: (source, preprocessor definitions).
        self.units = tuple((CSRC / source, defines) for source, defines in units)
        # Extra hipcc flags of those compilations.
        self.unit_flags = unit_flags

    def hip_compilations(self) -> list[tuple[Path, tuple[str, ...], str, tuple[str, ...]]]:
        """(source, definitions, object stem, extra flags) of every HIP compilation of this library."""

        out = [(self.hip_source, (), self.hip_source.stem, ())]
        for source, defines in self.units:
            suffix = "_".join(d.split("=", 1)[1] for d in defines)
            out.append((source, defines, f"{source.stem}_{suffix}", self.unit_flags))
        return out


LIBRARIES = (
    # The decode kernels compile once per (element type, head_dim), concurrently: one compilation of
    # every instantiation took about 7 minutes, a unit takes about one.
    Library("pa_decode_gfx950.hip", CABI_NAME, "pa_torch_ext.cpp", {EXTENSION_NAME: ("paged_attention_decode",)},
            units=tuple(("pa_decode_kernels.hip", (f"RK_PA_UNIT_ELEMENT={element}", f"RK_PA_UNIT_HEAD_DIM={head_dim}"))
                        for element in ("bf16", "fp16") for head_dim in (64, 128, 256)),
            # MFMA operands and results in architectural VGPRs: without it the compiler kept accumulators in
            # AGPRs and moved them for every VALU use (212 against 143 VALU per tile on the b128 kernel).
            # Measured with outputs bit-identical: the small workloads 1-4% faster, b128 unchanged, no
            # spills, and no kernel at lower occupancy (some at higher).
            unit_flags=("-mllvm", "-amdgpu-mfma-vgpr-form")),
    Library("kv_cache_gfx950.hip", "librk_kv_gfx950.so", "kv_torch_ext.cpp",
            {"rk_kv_append_gfx950": ("kv_cache_append",), "rk_kv_copy_gfx950": ("kv_cache_copy",)}),
    Library("sdpa_gfx950.hip", "librk_sdpa_gfx950.so", "sdpa_torch_ext.cpp", {"rk_sdpa_gfx950": ("sdpa",)}),
)


def compile_libraries(verbose: bool = False) -> dict[str, Path]:
    """Compile every C-ABI library (hipcc) and torch binding (g++); returns operator -> binding path."""

    import torch

    LIB_DIR.mkdir(parents=True, exist_ok=True)
    # A fixed build directory keeps the output byte-identical across builds: clang derives the
    # offload compilation-unit id from the command line, which includes the output path.
    work = PACKAGE_ROOT / "_build"
    work.mkdir(exist_ok=True)
    includes, libraries = _torch_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)

    # All compilations run concurrently; the library and the bindings are linked once the kernel
    # object exists.
    jobs = []
    for lib in LIBRARIES:
        hip = []
        for source, defines, stem, flags in lib.hip_compilations():
            obj = work / f"{stem}.o"
            hip.append((obj, _run([_hipcc(), *HIPCC_FLAGS, *flags, f"-I{INCLUDE}", *[f"-D{d}" for d in defines], "-c",
                                   str(source), "-o", str(obj)], verbose)))
        objects = {}
        for module in lib.bindings:
            ext_obj = work / f"{module}.o"
            cxx = [
                "g++",
                "-O2",
                "-std=c++17",
                "-fPIC",
                "-c",
                "-D__HIP_PLATFORM_AMD__=1",
                "-DUSE_ROCM=1",
                f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
                f"-DTORCH_EXTENSION_NAME={module}",
                "-DTORCH_API_INCLUDE_EXTENSION_H",
                f"-ffile-prefix-map={REPO_ROOT}=.",
                *[f"-I{path}" for path in includes],
                f"-I{sysconfig.get_paths()['include']}",
                f"-I{INCLUDE}",
                str(lib.binding_source),
                "-o",
                str(ext_obj),
            ]
            objects[module] = (ext_obj, _run(cxx, verbose))
        jobs.append((lib, hip, objects))

    rocm_lib = str(Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib")
    bindings: dict[str, Path] = {}
    for lib, hip, objects in jobs:
        for obj, process in hip:
            _finish(process, f"hipcc ({obj.stem})")
        kernel_objs = [str(obj) for obj, _ in hip]
        cabi_tmp = work / lib.cabi_name
        _finish(_run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *kernel_objs, "-Wl,--build-id=none",
                      "-o", str(cabi_tmp)], verbose), f"hipcc link ({lib.cabi_name})")
        linked = []
        for module, (ext_obj, gxx) in objects.items():
            _finish(gxx, f"g++ ({module} binding)")
            ext_tmp = work / f"{module}.so"
            link = [
                "g++",
                "-shared",
                str(ext_obj),
                *kernel_objs,
                *[f"-L{path}" for path in libraries],
                f"-L{rocm_lib}",
                "-lamdhip64",
                "-lc10",
                "-lc10_hip",
                "-ltorch",
                "-ltorch_cpu",
                "-ltorch_hip",
                "-ltorch_python",
                "-Wl,--build-id=none",
                "-o",
                str(ext_tmp),
            ]
            _finish(_run(link, verbose), f"link ({module} binding)")
            linked.append((module, ext_obj, ext_tmp))
        os.replace(cabi_tmp, LIB_DIR / lib.cabi_name)
        for module, ext_obj, ext_tmp in linked:
            os.replace(ext_tmp, LIB_DIR / f"{module}.so")
            ext_obj.unlink()
            for operator in lib.bindings[module]:
                bindings[operator] = LIB_DIR / f"{module}.so"
        for obj, _ in hip:
            obj.unlink()
    return bindings


def environment_record() -> dict:
    """Environment of the GPU this pack targets: gfx950 wave64 under the installed torch."""

    import torch

    sys.path.insert(0, str(PACKAGE_ROOT))
    from radeon_kernels.runtime.fingerprint import normalize_rocm_abi

    return {
        "architecture": ARCH,
        "wavefront_size": 64,
        "rocm_abi": normalize_rocm_abi(str(torch.version.hip)),
        "python_abi": f"cp{sys.version_info.major}{sys.version_info.minor}",
        "pytorch_version": str(torch.__version__),
    }


def write_pack_and_dispatch(bindings: dict[str, Path]) -> dict:
    sys.path.insert(0, str(PACKAGE_ROOT))
    from radeon_kernels.dispatch_plan import render_dispatch_manifest, render_pack_manifest

    digests = {operator: sha256_file(path) for operator, path in bindings.items()}
    environment = environment_record()
    pack = render_pack_manifest(environment=environment, digests=digests)
    _atomic_write(PACK_DIR / "manifest.json", json.dumps(pack, indent=2, sort_keys=True) + "\n")
    entries = {}
    for operator, digest in digests.items():
        dispatch = render_dispatch_manifest(operator, environment=environment, sha256=digest)
        target = PACKAGE_ROOT / "radeon_kernels" / "dispatch" / f"{operator}-1.0.json"
        _atomic_write(target, json.dumps(dispatch, indent=2, sort_keys=True) + "\n")
        entries[operator] = len(dispatch["entries"])
    return {"sha256": digests, "environment": environment, "entries": entries}


def compile_launch_loops(verbose: bool = False) -> Path:
    """The promotion timing's C launch loops (promotion/launch_loop.c): plain C, no GPU code."""

    source = PACKAGE_ROOT / "promotion" / "launch_loop.c"
    target = PACKAGE_ROOT / "promotion" / "liblaunch_loop.so"
    temporary = PACKAGE_ROOT / "_build" / "liblaunch_loop.so"
    temporary.parent.mkdir(exist_ok=True)
    _finish(_run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Werror", f"-ffile-prefix-map={REPO_ROOT}=.",
                  str(source), "-Wl,--build-id=none", "-o", str(temporary)], verbose), "gcc (launch_loop.c)")
    os.replace(temporary, target)
    return target


def build(verbose: bool = False) -> dict:
    compile_launch_loops(verbose)
    summary = write_pack_and_dispatch(compile_libraries(verbose=verbose))
    # Sign the pack manifest (the runtime loads only signed packs) and rewrite the promotion records
    # from the committed GPU evaluations (promotion/publish.py).
    sys.path.insert(0, str(PACKAGE_ROOT / "promotion"))
    from publish import publish

    summary["promotion"] = publish()
    if verbose:
        print(json.dumps(summary, indent=2), flush=True)
    return summary


if __name__ == "__main__":
    build(verbose="-v" in sys.argv or "--verbose" in sys.argv)
