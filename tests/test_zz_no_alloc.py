"""The allocation-free decode entry point (qh_flash_decode_noalloc) against the
workspace one (qh_flash_decode), called through the C ABI.

qh_flash_decode_noalloc keeps its split partials in a static device array, so
two calls in a row (the second on a smaller input) must each equal
qh_flash_decode's output and log-sum-exp bit for bit; a shape whose partials do
not fit the array is rejected before anything is launched.
"""
from __future__ import annotations

import pytest
import torch

from qwen_triton import _native

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, Hq, Hkv, cap, D, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    kc = torch.randn(B, Hkv, cap, D, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(B, Hkv, cap, D, generator=g).to(torch.bfloat16).to(DEV)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    return q, kc, vc


def _decode(name, q, k, v, seqlens, D):
    B, Hq = q.shape[:2]
    Hkv, Sk = k.shape[1], k.shape[2]
    out = torch.empty(B, Hq, 1, D, dtype=q.dtype, device=DEV)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=DEV)
    args = [q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), out.data_ptr(), lse.data_ptr(),
            None if seqlens is None else seqlens.data_ptr()]
    tail = [B, Hq, Hkv, Sk, D, D ** -0.5, _native.dtype_code(q.dtype), _native.stream(q.device)]
    if name == "qh_flash_decode":
        need = _native.call("qh_flash_decode_workspace", B, Hq, Hkv, Sk, D)
        ws = _native.workspace(need, q.device)
        _native.call(name, *args, ws.data_ptr(), ws.numel(), *tail)
    else:
        _native.call(name, *args, *tail)
    return out, lse


def test_flash_decode_noalloc_matches_workspace_entry():
    # first the config-3 shape (64 sequences x 8 kv heads, 2049 keys, GQA 2, per-sequence lengths:
    # the workgroup kernel, partials on chip, no scratch), then a larger split-KV call (8 sequences
    # x 8 kv heads, 2900 keys, GQA 4, per-sequence lengths), then a smaller one (1 sequence, 300
    # keys, GQA 2, no lengths): the last reuses the array the one before left filled
    cases = [(64, 16, 8, 2112, 2049, 128, True, 10), (8, 32, 8, 3000, 2900, 128, True, 11),
             (1, 16, 8, 320, 300, 128, False, 12)]
    for B, Hq, Hkv, cap, Sk, D, use_lens, seed in cases:
        print(f"[no_alloc] B={B} Hq={Hq} Hkv={Hkv} Sk={Sk} D={D} seqlens={use_lens}", flush=True)
        q, kc, vc = _inputs(B, Hq, Hkv, cap, D, seed)
        k, v = kc[:, :, :Sk], vc[:, :, :Sk]
        lens = None
        if use_lens:
            lens = torch.randint(0, Sk + 1, (B,), generator=torch.Generator().manual_seed(seed)).to(torch.int32)
            lens[0], lens[1] = 0, Sk
            lens = lens.to(DEV)
        c0 = _native.CALLS["qh_flash_decode_noalloc"]
        ref_o, ref_l = _decode("qh_flash_decode", q, k, v, lens, D)
        out_o, out_l = _decode("qh_flash_decode_noalloc", q, k, v, lens, D)
        torch.cuda.synchronize()
        assert _native.CALLS["qh_flash_decode_noalloc"] == c0 + 1
        assert torch.equal(out_o, ref_o)
        assert torch.equal(out_l, ref_l)


def test_flash_decode_noalloc_rejects_shapes_beyond_the_scratch():
    # head dim 64 with 4096 x 8 (sequence, kv-head) pairs and GQA 8: one split each, but
    # 4096 * 64 rows of 66 fp32 partials (69 MB) exceed the 16 MiB array; rejected on the host
    B, Hq, Hkv, Sk, D = 4096, 64, 8, 64, 64
    need = _native.call("qh_flash_decode_workspace", B, Hq, Hkv, Sk, D)
    assert need > 16 << 20
    with pytest.raises(_native.NativeError, match="static scratch"):
        _native.call("qh_flash_decode_noalloc", None, 0, 0, None, 0, 0, 0, None, 0, 0, 0, None, None, None,
                     B, Hq, Hkv, Sk, D, 0.125, _native.dtype_code(torch.bfloat16), _native.stream(torch.device(DEV)))
