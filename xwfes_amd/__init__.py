"""MI355X-native speculative-decoding verify path (HIP kernels for gfx950
behind the C ABI of include/ftx.h).  `xwfes_amd.ftx` is the ctypes binding;
`xwfes_amd.synth` builds synthetic GGUF-shaped models on the device."""
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_PATH = os.path.join(PKG_DIR, "libftx.so")


def build(jobs=8):
    """Compile libftx.so for gfx950 from csrc/ (always recompiles)."""
    import subprocess
    subprocess.check_call(["make", "-s", "-C", CSRC, "clean"])
    subprocess.check_call(["make", "-s", "-j%d" % jobs, "-C", CSRC])
    return LIB_PATH
