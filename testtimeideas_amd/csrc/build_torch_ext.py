"""Build testtimeideas_amd/_ttt_torch.so, the torch binding of the C entry
points (ttt_torch.cpp), against the in-tree libttt_attn.so (found next
to the module through an $ORIGIN run path).  The object goes to _build/ext.
Run after the library is built (``make -C testtimeideas_amd/csrc``)."""
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
NAME = "_ttt_torch"


def build(verbose: bool = False) -> str:
    from torch.utils import cpp_extension

    out_dir = os.path.join(ROOT, "_build", "ext")
    os.makedirs(out_dir, exist_ok=True)
    obj = os.path.join(out_dir, "ttt_torch.o")
    dst = os.path.join(PKG, NAME + ".so")
    inc = [f"-I{p}" for p in cpp_extension.include_paths()] + [f"-I{sysconfig.get_paths()['include']}",
                                                              "-I/opt/rocm/include"]
    cflags = ["-O2", "-fPIC", "-std=c++17", f"-DTORCH_EXTENSION_NAME={NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
              "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1"]
    compile_cmd = ["c++", *cflags, *inc, "-c", os.path.join(HERE, "ttt_torch.cpp"), "-o", obj]
    libs = [f"-L{p}" for p in cpp_extension.library_paths()]
    link_cmd = ["c++", "-shared", obj, "-o", dst + ".tmp", f"-L{PKG}", "-lttt_attn", "-Wl,-rpath,$ORIGIN", *libs,
                "-lc10_hip", "-lc10", "-ltorch_cpu", "-ltorch", "-ltorch_python"]
    for cmd in (compile_cmd, link_cmd):
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
    os.replace(dst + ".tmp", dst)
    return dst


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
