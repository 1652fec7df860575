"""launch_glint_htile_bf16_stream_noalloc: the BF16-out H-TILE with its split-K partials
and counters in the library's static per-device scratch instead of a workspace it
allocates. Called through the C ABI and checked bit for bit against
launch_glint_htile_bf16_stream (same kernels, same split plan), on two calls in a row,
the second with a smaller input, and on a shape that does not split."""
import pytest

from glint_amd import glint_hip as H
from tests.gpu_util import torch_cuda

pytestmark = pytest.mark.gpu


def _pin(torch, N, K, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(N * K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    return H.encode_bf16(w, 64)


def _call(torch, fn, pin, x, N, K):
    M = x.shape[0]
    y = torch.full((M, N), -1, dtype=torch.int16, device="cuda")
    rc = fn(H._p(pin[0]), H._p(pin[1]), H._p(pin[2]), H._p(x), H._p(y), M, N, K, 64, H._stream())
    assert rc == 0, rc
    return y


def test_noalloc_matches_allocating_entry():
    torch = torch_cuda()
    lib = H.encode_lib()
    ref_fn, na_fn = lib.launch_glint_htile_bf16_stream, lib.launch_glint_htile_bf16_stream_noalloc
    g = torch.Generator(device="cuda").manual_seed(7)
    for M, N, K in [(1024, 4096, 14336), (512, 4096, 14336), (64, 4096, 4096), (2048, 384, 640), (1, 1024, 4096)]:
        print(f"noalloc M={M} N={N} K={K}", flush=True)
        pin = _pin(torch, N, K, 11 + N + K)
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        want = _call(torch, ref_fn, pin, x, N, K)
        got = _call(torch, na_fn, pin, x, N, K)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, N, K)
    rc = na_fn(None, None, None, None, None, 4, 4, 64, 64, H._stream())
    assert rc == -1
