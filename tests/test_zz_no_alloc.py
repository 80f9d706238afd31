"""flyai_linear_bf16_noalloc: the linear whose split-K partials live in the library's static device
array instead of a caller workspace.  Through the C ABI it must give the workspace entry point's
exact bits, call after call on one GPU, including a call with a smaller input right after a larger
one (the array keeps the previous call's partials, which must never leak into the next result).
Shapes past the array's 16 MiB are refused on the host before anything is launched."""
import ctypes as C

import pytest
import torch

from flyai_amd import _lib

DEV = "cuda"


def _p(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _inputs(M, N, K, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(N, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    res = torch.randn(M, N, device=DEV, generator=g).to(torch.bfloat16)
    return x, w, b, res


def _with_workspace(lib, x, w, b, M, N, K, residual):
    ws = torch.empty(int(lib.flyai_linear_workspace_bytes(M, N, K)) // 4 + 1, dtype=torch.float32, device=DEV)
    y = None if residual is not None else torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.flyai_linear_bf16(_p(x), _p(w), _p(b), M, N, K, _p(y), _p(residual), _p(ws), _stream()))
    return residual if residual is not None else y


def _no_alloc(lib, x, w, b, M, N, K, residual):
    y = None if residual is not None else torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.flyai_linear_bf16_noalloc(_p(x), _p(w), _p(b), M, N, K, _p(y), _p(residual), _stream()))
    return residual if residual is not None else y


# (M, N, K, with residual): pairs of consecutive calls, the second one smaller -- split-K with 6 and 8
# partial planes, and the tiled kernel's one plane from 256 rows
PAIRS = [
    ((48, 5120, 2880, False), (5, 5120, 2880, False)),
    ((64, 2880, 4096, True), (7, 2880, 4096, True)),
    ((300, 2880, 4096, False), (256, 512, 2880, True)),
]


@pytest.mark.gpu
@pytest.mark.parametrize("first,second", PAIRS)
def test_linear_noalloc_matches_workspace_linear(first, second):
    lib = _lib.lib()
    for i, (M, N, K, with_res) in enumerate((first, second)):
        x, w, b, res = _inputs(M, N, K, 100 * i + M)
        want = _with_workspace(lib, x, w, b, M, N, K, res.clone() if with_res else None)
        got = _no_alloc(lib, x, w, b, M, N, K, res.clone() if with_res else None)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i} (M={M} N={N} K={K} residual={with_res}): bits differ"


def test_linear_noalloc_refuses_shapes_past_its_scratch():
    lib = _lib.lib()
    assert lib.flyai_linear_noalloc_max_bytes() == 16 << 20
    # 2048 rows take the tiled kernel's single plane: 2048 * 5120 * 4 bytes = 40 MiB > 16 MiB
    fake = C.c_void_p(0x100000)
    rc = lib.flyai_linear_bf16_noalloc(fake, fake, fake, 2048, 5120, 2880, fake, None, None)
    assert rc == _lib.FLYAI_EINVAL and b"static scratch" in lib.flyai_last_error()
    # 64 rows of split-K over K = 8192 (16 planes) at N = 5120: 20 MiB
    rc = lib.flyai_linear_bf16_noalloc(fake, fake, fake, 64, 5120, 8192, fake, None, None)
    assert rc == _lib.FLYAI_EINVAL
