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


# ------------------------------------------------------------------------------------------
# fp8 e4m3 (OCP) and the VSL_DT_F16F8 activation form, in numpy: the values the GEMM's fp8 lo path is
# defined to multiply (the lo plane, and B rounded to e4m3 as B * 2^s)
# ------------------------------------------------------------------------------------------
def e4m3_table():
    """Value of every byte code (NaN for 0x7f / 0xff)."""
    c = np.arange(256)
    e, m, s = (c >> 3) & 15, c & 7, np.where(c >> 7, -1.0, 1.0)
    v = np.where(e > 0, np.ldexp(1.0 + m / 8.0, e - 7), np.ldexp(m / 8.0, -6)) * s
    v[0x7F] = v[0xFF] = np.nan
    return v


def e4m3_encode(x):
    """Codes of the nearest e4m3 values (ties to the even code, magnitudes above 448 saturate, the sign
    of a zero result kept)."""
    x = np.asarray(x, np.float64)
    pos = e4m3_table()[:127]                  # codes 0..126, increasing
    a = np.minimum(np.abs(x), 448.0)
    i = np.clip(np.searchsorted(pos, a), 1, 126)
    lo, hi = pos[i - 1], pos[i]
    take_hi = (a - lo > hi - a) | ((a - lo == hi - a) & (i % 2 == 0))
    code = np.where(take_hi, i, i - 1).astype(np.uint8)
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)


def lo8_perm(K):
    """Position of column k inside its row of the lo8 plane (bits 3 and 4 of k exchanged)."""
    k = np.arange(K)
    return (k & ~24) | ((k & 8) << 1) | ((k & 16) >> 1)


def f16f8_split(a):
    """VSL_DT_F16F8 planes of fp32 rows a [M][K]: (hi fp16 [M][K], lo8 bytes [M][K] in the plane's
    order, the value hi + lo8 * 2^-12 as float64)."""
    a = np.asarray(a, np.float32)
    hi = a.astype(np.float16)
    lo = (a - hi.astype(np.float32)).astype(np.float64) * 4096.0
    codes = e4m3_encode(lo)
    val = hi.astype(np.float64) + e4m3_table()[codes] / 4096.0
    plane = np.empty_like(codes)
    plane[:, lo8_perm(a.shape[1])] = codes
    return hi, plane, val


def f16f8_value(hi, plane):
    """hi + lo8 * 2^-12 of stored planes (plane in its stored order)."""
    codes = plane[:, lo8_perm(plane.shape[1])]
    return hi.astype(np.float64) + e4m3_table()[codes] / 4096.0


def f8lo_product(hi, lo_val, B, shift=6):
    """What a GEMM with an F16F8 A computes: hi B^T + lo B8^T, B8 = e4m3(B * 2^s) / 2^s (float64), s the
    weight shift (VSL_GEMM_B8_SHIFT; 6 without one)."""
    B8 = e4m3_table()[e4m3_encode(np.ldexp(B.astype(np.float64), shift))]
    return hi.astype(np.float64) @ B.astype(np.float64).T + lo_val @ np.ldexp(B8, -shift).T


def b8_shift_model(max_abs):
    """The weight shift for a matrix whose largest finite magnitude is max_abs, by search: the largest s
    in [-16, 30] with max_abs * 2^s <= 448 (6 for 0 or a non-finite value)."""
    m = float(max_abs)
    if not (m > 0) or not np.isfinite(m):
        return 6
    ok = [s for s in range(-16, 31) if np.ldexp(np.float32(m), s) <= 448.0]
    return max(ok) if ok else -16
