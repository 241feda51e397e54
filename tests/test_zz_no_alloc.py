"""GPU: ``asrattn_decode_noalloc`` (split partials in the library's static
device array) against ``asrattn_decode`` with a caller-owned workspace, both
called through the C ABI.

Bar: bit-identical outputs (the same kernels with the same split count; only
where the partials live differs), on two calls in a row, the second with a
smaller input so that it runs over what the first left in the array.  A
float32 torch reference checks that the shared result is the attention
(1e-5 for f32, 2e-2 for bf16, relative to max |ref|).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import assert_close

pytestmark = pytest.mark.gpu

KIND = {torch.float32: "f32", torch.bfloat16: "bf16"}


def say(*args):
    print(*args, flush=True)


def case(batch, heads_q, heads_kv, head_dim, length, dtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(batch, heads_q, head_dim, generator=g).to("cuda", dtype)
    k = torch.randn(batch, length, heads_kv, head_dim, generator=g).to("cuda", dtype)
    v = torch.randn(batch, length, heads_kv, head_dim, generator=g).to("cuda", dtype)
    # Ragged key counts, the shortest 1 and the longest the full length.
    used = torch.randint(1, length + 1, (batch,), generator=g, dtype=torch.int32)
    used[0], used[-1] = length, 1
    return q, k, v, used.to("cuda")


def reference(q, k, v, used):
    qf, kf, vf = q.float().cpu(), k.float().cpu(), v.float().cpu()
    group = q.shape[1] // k.shape[2]
    out = torch.empty_like(qf)
    for b, n in enumerate(used.cpu().tolist()):
        kk = kf[b, :n].repeat_interleave(group, dim=1).transpose(0, 1)  # (heads_q, n, d)
        vv = vf[b, :n].repeat_interleave(group, dim=1).transpose(0, 1)
        s = torch.einsum("hd,hnd->hn", qf[b], kk) / q.shape[2] ** 0.5
        out[b] = torch.einsum("hn,hnd->hd", torch.softmax(s, dim=-1), vv)
    return out


def run_both(q, k, v, used):
    from asrback_amd import _lib, attention

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    out_ws = torch.full_like(q, float("nan"))
    out_na = torch.full_like(q, float("nan"))
    params = attention._decode_params(q, k, v, out_ws, used, None, 0, None)
    splits = lib.asrattn_decode_num_splits(ctypes.byref(params))
    need = lib.asrattn_decode_workspace_size(ctypes.byref(params))
    assert splits > 1 and 0 < need <= 8 << 20, (splits, need)
    workspace = torch.empty(need, dtype=torch.uint8, device="cuda")
    _lib.check(lib.asrattn_decode(ctypes.byref(params), workspace.data_ptr(), need, stream), "asrattn_decode")
    params.out = out_na.data_ptr()
    _lib.check(lib.asrattn_decode_noalloc(ctypes.byref(params), stream), "asrattn_decode_noalloc")
    torch.cuda.synchronize()
    return out_ws, out_na, splits


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_decode_on_two_calls(dtype):
    # First call: 2 x 4 kv heads over 4096 keys, 16 query heads of 128
    # (16 splits); second: 1 x 2 kv heads over 700 keys, 8 heads of 64
    # (3 splits), over the partials the first call left behind.
    shapes = [(2, 16, 4, 128, 4096, 11), (1, 8, 2, 64, 700, 12)]
    for batch, hq, hkv, hd, length, seed in shapes:
        say(f"noalloc dtype={dtype} batch={batch} heads={hq}/{hkv} head_dim={hd} length={length} seed={seed}")
        q, k, v, used = case(batch, hq, hkv, hd, length, dtype, seed)
        out_ws, out_na, splits = run_both(q, k, v, used)
        assert torch.equal(out_na, out_ws), f"{splits} splits: noalloc differs from decode with a workspace"
        assert_close(out_na.float().cpu(), reference(q, k, v, used), KIND[dtype], label=f"noalloc {dtype} hd{hd}")


def test_noalloc_rejects_oversize_and_keeps_working():
    from asrback_amd import _lib, attention

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    q, k, v, used = case(1, 8, 1, 256, 2048, torch.bfloat16, 13)
    out = torch.zeros_like(q)
    params = attention._decode_params(q, k, v, out, used, None, 1024, None)
    say("noalloc oversize: num_splits=1024 head_dim=256")
    assert lib.asrattn_decode_noalloc(ctypes.byref(params), stream) == _lib.ERR_WORKSPACE
    assert b"scratch" in lib.asrattn_last_error()
    torch.cuda.synchronize()
    assert not out.any()  # nothing was launched
    params.num_splits = 0
    _lib.check(lib.asrattn_decode_noalloc(ctypes.byref(params), stream), "asrattn_decode_noalloc")
    torch.cuda.synchronize()
    assert_close(out.float().cpu(), reference(q, k, v, used), "bf16", label="noalloc after rejection")
