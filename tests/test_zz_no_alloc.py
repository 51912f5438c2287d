"""vsl_attn_decode_noalloc (split partials in the library's static device array, no workspace
argument, no allocation) against vsl_attn_decode with a caller workspace, through the C ABI: equal bit
for bit on two calls in a row, the second with a smaller input, and the size limits refused."""
import math

import numpy as np
import pytest

import vsl_testlib

pytestmark = pytest.mark.gpu


def _case(vsl, H, dev, nq, nkv, hd, kvdt, cap, length, nsplit, seed):
    rng = np.random.default_rng(seed)
    kvnp = np.float16 if kvdt == 1 else np.float32
    K = rng.normal(0, 1, (nkv, cap, hd)).astype(kvnp)
    V = rng.normal(0, 1, (nkv, cap, hd)).astype(kvnp)
    K[:, length:] = np.nan  # never written: must not reach the output
    V[:, length:] = np.nan
    q = rng.normal(0, 1, nq * hd).astype(np.float32)
    dq, dk, dv = dev.put(q), dev.put(K), dev.put(V)
    scale = 1.0 / math.sqrt(hd)
    ctrl = dev.empty((8,), np.int32)
    vsl.check(H.vsl_ctrl_reset(dev.p(ctrl), length - 1, 4, 0, cap, None))
    po = dev.empty((nq * nsplit * hd,), np.float32)
    pml = dev.empty((nq * nsplit * 2,), np.float32)
    ref = dev.empty((nq * hd,), np.float32)
    vsl.check(H.vsl_attn_decode(dev.p(dq), dev.p(dk), dev.p(dv), kvdt, nq, nkv, hd, cap, scale, nsplit, dev.p(po),
                                dev.p(pml), dev.p(ref), dev.p(ctrl), None))
    out = dev.empty((nq * hd,), np.float32)
    vsl.check(H.vsl_attn_decode_noalloc(dev.p(dq), dev.p(dk), dev.p(dv), kvdt, nq, nkv, hd, cap, scale, nsplit,
                                        dev.p(out), dev.p(ctrl), None))
    r, o = dev.get(ref), dev.get(out)
    assert np.all(np.isfinite(o))
    assert np.array_equal(o.view(np.uint32), r.view(np.uint32))


def test_attn_decode_noalloc_matches_workspace_entry():
    vsl = vsl_testlib.package()
    H = vsl.hip()
    dev = vsl_testlib.Dev()
    try:
        # 8B layout at the full partials budget (32 heads x 128 splits = 4096 pairs), then a smaller
        # call (fewer heads, splits and positions, head_dim 64, fp32 cache): the second call reuses the
        # array the first one filled
        _case(vsl, H, dev, nq=32, nkv=8, hd=128, kvdt=1, cap=2048, length=1500, nsplit=128, seed=1)
        _case(vsl, H, dev, nq=4, nkv=4, hd=64, kvdt=0, cap=512, length=37, nsplit=7, seed=2)
        # the matrix-core kernel (fp16, head_dim 128, capacity above 8192)
        _case(vsl, H, dev, nq=32, nkv=8, hd=128, kvdt=1, cap=16384, length=9000, nsplit=32, seed=3)
        # beyond the static array: refused before any launch
        q = dev.empty((64 * 128,), np.float32)
        out = dev.empty((64 * 128,), np.float32)
        ctrl = dev.empty((8,), np.int32)
        kv = dev.empty((8 * 64 * 256,), np.float16)
        assert H.vsl_attn_decode_noalloc(dev.p(q), dev.p(kv), dev.p(kv), 1, 64, 8, 128, 64, 0.1, 65, dev.p(out),
                                         dev.p(ctrl), None) == -104
        assert H.vsl_attn_decode_noalloc(dev.p(q), dev.p(kv), dev.p(kv), 1, 8, 8, 256, 64, 0.1, 4, dev.p(out),
                                         dev.p(ctrl), None) == -104
        assert "static partials buffer" in vsl.hip().vsl_last_error().decode()
    finally:
        dev.release()
