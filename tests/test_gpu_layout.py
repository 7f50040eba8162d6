"""Device check of the 32x32 MFMA operand/result layout the kernels are built on
(elsa_mfma.h): A[i][k] in lane i + 32*(k / KP), B[k][j] in lane j + 32*(k / KP),
D[i][j] in lane j + 32*g, register (i/8)*4 + (i%4) with g = (i/4)%2."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from elsa_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("variant,kp,dt", [(0, 8, torch.float16), (1, 8, torch.bfloat16), (2, 1, torch.float32)])
def test_mfma_32x32_layout(variant, kp, dt):
    print(f"mfma layout variant={variant}", flush=True)
    kdim = 2 * kp
    rng = np.random.default_rng(variant)
    A = rng.integers(-4, 5, size=(32, kdim)).astype(np.float32)
    B = rng.integers(-4, 5, size=(kdim, 32)).astype(np.float32)
    a_l = np.zeros((64, kp), np.float32)
    b_l = np.zeros((64, kp), np.float32)
    for lane in range(64):
        c, g = lane % 32, lane // 32
        for t in range(kp):
            a_l[lane, t] = A[c, g * kp + t]
            b_l[lane, t] = B[g * kp + t, c]
    a_t = torch.from_numpy(a_l).to("cuda", dt).contiguous()
    b_t = torch.from_numpy(b_l).to("cuda", dt).contiguous()
    d_t = torch.zeros(64 * 16, dtype=torch.float32, device="cuda")
    lib = _lib.load()
    _lib.check(lib.elsa_debug_mfma(variant, a_t.data_ptr(), b_t.data_ptr(), d_t.data_ptr(),
                                   _lib.stream_handle(a_t.device)), "elsa_debug_mfma")
    torch.cuda.synchronize()
    d = d_t.cpu().numpy().reshape(64, 16)
    ref = A @ B
    got = np.zeros((32, 32), np.float32)
    for lane in range(64):
        c, g = lane % 32, lane // 32
        for r in range(16):
            got[(r // 4) * 8 + 4 * g + (r % 4), c] = d[lane, r]
    np.testing.assert_array_equal(got, ref)
