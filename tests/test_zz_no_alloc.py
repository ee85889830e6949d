"""fa_fwd_noalloc: the forward that allocates nothing (split-KV partials in a
device array inside the library) against fa_fwd_ws with a caller workspace,
called through the C ABI.

The GPU test runs two decoding shapes that take the split path, the second
smaller than the first, so the second call runs on the array the first left
behind, then a causal launch whose key ranges cover the keys its queries see;
each result must equal fa_fwd_ws's bit for bit (same kernels, same
split, same summation order) and match the fp64 oracle at the north-star
tolerances. The CPU test checks the size limit, which is enforced before any
HIP call.
"""

from __future__ import annotations

import ctypes
import json
import sys

import numpy as np
import pytest
import torch

from fa_testutil import LSE_TOL, assert_close, make_inputs
from oracle import oracle
from triton_flash_attention import _lib

# (B, Hq, Hkv, N_q, N_kv, D, causal); all take the split-KV forward.
NOALLOC_CASES = [
    (2, 8, 2, 3, 6000, 128, False),
    (1, 4, 1, 2, 3000, 64, False),  # smaller: fewer partials than the call before
    (1, 2, 1, 2100, 2400, 32, True),  # causal: ranges over the 2100 visible keys
]


def _note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def test_noalloc_rejects_partials_beyond_the_scratch():
    lib = _lib.load()
    limit = lib.fa_fwd_noalloc_max_workspace_bytes()
    assert limit == 64 << 20
    # 511 query heads x one 128-query tile: 511 work-groups, split in two ranges.
    shape = (1, 511, 1, 128, 4096, 128)
    need = lib.fa_fwd_workspace_bytes(*shape, 0)
    assert need > limit
    fake = ctypes.c_void_p(0x10000)  # never dereferenced: rejected before any HIP call
    rc = lib.fa_fwd_noalloc(fake, fake, fake, fake, fake, *shape, 128 ** -0.5, 0, None)
    assert rc == _lib.FA_ERR_TOO_LARGE
    msg = _lib.last_error()
    assert "fa_fwd_noalloc" in msg and str(need) in msg and str(limit) in msg
    # A bad argument is rejected the same way as by fa_fwd_ws.
    assert lib.fa_fwd_noalloc(fake, fake, fake, fake, fake, 1, 4, 1, 2, 3000, 64, -1.0, 1,
                              None) == _lib.FA_ERR_BAD_SCALE


@pytest.mark.gpu
def test_noalloc_forward_matches_workspace_forward_twice():
    lib = _lib.load()
    dev = torch.device("cuda")
    for B, Hq, Hkv, N, Nkv, D, causal in NOALLOC_CASES:
        tag = f"noalloc fwd B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={D} causal={causal}"
        _note(tag)
        need = lib.fa_fwd_workspace_bytes(B, Hq, Hkv, N, Nkv, D, int(causal))
        assert 0 < need <= lib.fa_fwd_noalloc_max_workspace_bytes(), tag
        q, k, v, _ = make_inputs(B, Hq, Hkv, N, D, seed=7 * N + Nkv + D, n_kv=Nkv)
        qd, kd, vd = (t.to(dev) for t in (q, k, v))
        scale = D ** -0.5
        stream = torch.cuda.current_stream().cuda_stream
        o_ws, o_na = torch.empty_like(qd), torch.empty_like(qd)
        lse_ws = torch.empty((B, Hq, N), device=dev, dtype=torch.float32)
        lse_na = torch.empty_like(lse_ws)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        _lib.check(lib.fa_fwd_ws(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o_ws.data_ptr(),
                                 lse_ws.data_ptr(), B, Hq, Hkv, N, Nkv, D, scale, int(causal),
                                 ws.data_ptr(), need, stream))
        _lib.check(lib.fa_fwd_noalloc(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                      o_na.data_ptr(), lse_na.data_ptr(), B, Hq, Hkv, N, Nkv, D,
                                      scale, int(causal), stream))
        torch.cuda.synchronize()
        assert torch.equal(o_na, o_ws), f"{tag}: O differs from fa_fwd_ws"
        assert torch.equal(lse_na, lse_ws), f"{tag}: LSE differs from fa_fwd_ws"
        o_ref, lse_ref = oracle.fwd(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                    causal, scale)
        assert_close(f"{tag} o", o_na.double().cpu().numpy(), o_ref)
        lse_err = float(np.max(np.abs(lse_na.double().cpu().numpy() - lse_ref)))
        assert lse_err <= LSE_TOL, f"{tag} lse {lse_err:.3e}"
        _note(f"{tag}: equal to fa_fwd_ws, lse err {lse_err:.2e}, partials {need} bytes")


# Run in a fresh process: free device memory around loading the library, a
# plain forward and the first fa_fwd_noalloc (inputs allocated beforehand, so
# the caching allocator takes nothing in between).
_RESIDENCY_SCRIPT = r'''
import json, sys
sys.path.insert(0, sys.argv[1])
import torch
dev = torch.device("cuda")
small = [torch.randn(1, 2, 64, 64, device=dev).half() for _ in range(3)]
o_s, lse_s = torch.empty_like(small[0]), torch.empty(1, 2, 64, device=dev)
B, Hq, Hkv, N, Nkv, D = 2, 8, 2, 3, 6000, 128
q = torch.randn(B, Hq, N, D, device=dev).half()
k = torch.randn(B, Hkv, Nkv, D, device=dev).half()
v = torch.randn(B, Hkv, Nkv, D, device=dev).half()
o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=dev)
torch.cuda.synchronize()
free = lambda: torch.cuda.mem_get_info()[0]
r = [free()]
from triton_flash_attention import _lib
lib = _lib.load()
torch.cuda.synchronize()
r.append(free())
s = torch.cuda.current_stream().cuda_stream
_lib.check(lib.fa_fwd(*(t.data_ptr() for t in small), o_s.data_ptr(), lse_s.data_ptr(),
                      1, 2, 2, 64, 64, 0.125, 1, s))
torch.cuda.synchronize()
r.append(free())
_lib.check(lib.fa_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                              lse.data_ptr(), B, Hq, Hkv, N, Nkv, D, D ** -0.5, 0, s))
torch.cuda.synchronize()
r.append(free())
print("RESULT " + json.dumps(r), flush=True)
'''


@pytest.mark.gpu
def test_noalloc_scratch_is_reserved_at_the_first_noalloc_call():
    """The 64 MiB array sits in a code object with no kernel, so under HIP's
    default deferred code-object loading a process that only loads the
    library and runs plain launches does not hold it; the first
    fa_fwd_noalloc on the GPU does. Measured with hipMemGetInfo in a fresh
    process (the environment's HIP_ENABLE_DEFERRED_LOADING is left as is)."""
    import os
    import subprocess
    from pathlib import Path

    pkg = Path(__file__).resolve().parent.parent / "triton-flash-attention_amd"
    env = {k: v for k, v in os.environ.items() if k != "HIP_ENABLE_DEFERRED_LOADING"}
    p = subprocess.run([sys.executable, "-c", _RESIDENCY_SCRIPT, str(pkg)], capture_output=True,
                       text=True, timeout=240, env=env)
    line = [ln for ln in p.stdout.splitlines() if ln.startswith("RESULT ")]
    assert p.returncode == 0 and line, p.stdout[-2000:] + p.stderr[-2000:]
    start, loaded, after_fwd, after_noalloc = json.loads(line[0][7:])
    MiB = 1 << 20
    _note(f"free-memory drops: dlopen {(start - loaded) / MiB:.0f} MiB, first fa_fwd "
          f"{(loaded - after_fwd) / MiB:.0f} MiB, first fa_fwd_noalloc "
          f"{(after_fwd - after_noalloc) / MiB:.0f} MiB")
    limit = _lib.load().fa_fwd_noalloc_max_workspace_bytes()
    assert start - after_fwd < limit // 2, "loading and a plain forward reserved the scratch"
    assert after_fwd - after_noalloc >= limit, "the first fa_fwd_noalloc did not reserve it"
