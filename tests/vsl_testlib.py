"""Shared helpers for the tests: import the package (its directory name has dashes), the oracle,
and device buffers for kernel-level GPU tests (torch is used only as device-memory plumbing)."""
import importlib.util
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "vulkan-symbiote-loader_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def ensure_built():
    libs = [os.path.join(PKG_DIR, "lib", "libvsl_hip.so"), os.path.join(PKG_DIR, "lib", "libvsl_engine.so")]
    if not all(os.path.exists(p) for p in libs):
        subprocess.run([sys.executable, os.path.join(PKG_DIR, "build.py")], check=True)
    if not os.path.exists(os.path.join(ROOT, "oracle", "libvsl_oracle.so")):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, stdout=subprocess.DEVNULL)


def package():
    name = "vulkan_symbiote_loader_amd"
    if name in sys.modules:
        return sys.modules[name]
    ensure_built()
    spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def oracle():
    ensure_built()
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    return orc


class Dev:
    """Device buffers through torch (plumbing only); pointers go to the C ABI."""

    def __init__(self):
        import torch
        self.torch = torch
        assert torch.cuda.is_available(), "GPU tests need a HIP device"
        self.dev = torch.device("cuda:0")
        # every buffer stays referenced until release(): a pointer handed to the C ABI must not
        # outlive its tensor (torch's caching allocator reuses freed blocks at once)
        self._live = []

    def release(self):
        self.torch.cuda.synchronize()
        self._live = []

    def put(self, a):
        t = self.torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)
        self._live.append(t)
        return t

    def empty(self, shape, dtype):
        tdt = {np.float32: self.torch.float32, np.float16: self.torch.float16, np.uint32: self.torch.int32,
               np.int32: self.torch.int32, np.uint8: self.torch.uint8}[np.dtype(dtype).type]
        t = self.torch.zeros(shape, dtype=tdt, device=self.dev)
        self._live.append(t)
        return t

    @staticmethod
    def p(t):
        return None if t is None else t.data_ptr()

    def get(self, t, dtype=None):
        self.torch.cuda.synchronize()
        a = t.cpu().numpy()
        if dtype is not None:
            a = a.view(dtype)
        return a

    def sync(self):
        self.torch.cuda.synchronize()
