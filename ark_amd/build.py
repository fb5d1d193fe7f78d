"""Build the gfx950 library (hipcc via ark_amd/csrc/Makefile)."""
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))


def build(force=True, arch="gfx950"):
    """Compile ark_amd/lib/libark_opt.so; force=True rebuilds every time."""
    cmd = ["make", "-C", os.path.join(_HERE, "csrc"), f"ARCH={arch}"]
    if force:
        cmd.insert(1, "-B")
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc build failed:\n" + r.stdout[-4000:])
    return os.path.join(_HERE, "lib", "libark_opt.so")
