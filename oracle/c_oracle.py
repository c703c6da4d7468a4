"""TEST INFRASTRUCTURE ONLY: ctypes wrapper of oracle/quant_ref.c (built by `make -C oracle`)."""
import ctypes
import os
import subprocess

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "build", "liboracle_quant.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


def codes(x, s):
    """sat127(rintf(x / s)) elementwise; x, s float32 tensors of equal size."""
    x = np.ascontiguousarray(x.float().numpy())
    s = np.ascontiguousarray(s.float().numpy())
    out = np.empty(x.size, dtype=np.int8)
    lib().oracle_codes(_p(x), _p(s), ctypes.c_int64(x.size), ctypes.c_int64(s.size), _p(out))
    return torch.from_numpy(out.reshape(x.shape))


def quant_rows(x_bf16, mu, s):
    """x bf16 [rows, H, D]; mu float32 [H, D] or None; s float32 [H, D] or [H, 1] -> int8 codes."""
    rows, H, D = x_bf16.shape
    xb = np.ascontiguousarray(x_bf16.contiguous().view(torch.int16).numpy())
    sb = np.ascontiguousarray(s.float().numpy())
    mb = np.ascontiguousarray(mu.float().numpy()) if mu is not None else None
    out = np.empty((rows, H, D), dtype=np.int8)
    lib().oracle_quant_rows(_p(xb), _p(mb) if mb is not None else None, _p(sb), ctypes.c_int64(rows),
                            ctypes.c_int64(H), ctypes.c_int64(D), ctypes.c_int64(s.shape[-1]), _p(out))
    return torch.from_numpy(out)


def dequant(q, s):
    """int8 [rows, H, D] x scales [H, D] or [H, 1] -> bf16 (fp32 product, RNE)."""
    rows, H, D = q.shape
    qb = np.ascontiguousarray(q.numpy())
    sb = np.ascontiguousarray(s.float().numpy())
    out = np.empty((rows, H, D), dtype=np.int16)
    lib().oracle_dequant(_p(qb), _p(sb), ctypes.c_int64(rows), ctypes.c_int64(H), ctypes.c_int64(D),
                         ctypes.c_int64(s.shape[-1]), _p(out))
    return torch.from_numpy(out).view(torch.bfloat16)


def quant_q(q, ks, group):
    """q bf16 [T, Hq, D], ks [Hkv, D] or [Hkv, 1] -> (codes [T, Hq, D], scales [T, Hq, D / group])."""
    T, hq, D = q.shape
    hkv = ks.shape[0]
    qb = np.ascontiguousarray(q.contiguous().view(torch.int16).numpy())
    kb = np.ascontiguousarray(ks.float().numpy())
    codes_ = np.empty((T, hq, D), dtype=np.int8)
    sc = np.empty((T, hq, D // group), dtype=np.float32)
    lib().oracle_quant_q(_p(qb), _p(kb), ctypes.c_int64(T * hq), ctypes.c_int64(hq), ctypes.c_int64(hq // hkv),
                         ctypes.c_int64(D), ctypes.c_int64(ks.shape[-1]), ctypes.c_int64(group), _p(codes_), _p(sc))
    return torch.from_numpy(codes_), torch.from_numpy(sc)
