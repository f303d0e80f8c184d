"""mlxr_moe_block_forward_noalloc (the block forward whose scratch is the
library's own per-GPU device array) against mlxr_moe_block_forward with a
caller workspace, through the C ABI: the same kernels on the same values,
so outputs and routing are bit-identical.  Calls in a row, each with
fewer tokens than the last (the array keeps the previous call's contents;
T = 1 takes the down launch that carries the combine), and a T whose
workspace exceeds the array is refused on the host."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _noalloc(pkg, block, x, T):
    C = pkg._capi
    d = block.hidden_size
    out = torch.empty((T, d), dtype=block.out_dtype, device=x.device)
    idx = torch.empty((T, block.num_experts_per_tok), dtype=torch.int32, device=x.device)
    wts = torch.empty((T, block.num_experts_per_tok), dtype=torch.float32, device=x.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    C.check(C.lib().mlxr_moe_block_forward_noalloc(
        ctypes.byref(block.descriptor()), x.data_ptr(), T, out.data_ptr(), idx.data_ptr(),
        wts.data_ptr(), stream))
    return out, idx, wts


@pytest.mark.parametrize("cfg", ["c2", "c4", "c6"])
def test_noalloc_block_equals_workspace_block(pkg, dev, cfg):
    W = pkg.workloads
    bw = W.make_weights(W.CONFIGS[cfg], dev)
    block = bw.block()
    lib = pkg._capi.lib()
    assert lib.mlxr_moe_noalloc_scratch_size() == 32 * 1024 * 1024
    for T in (64, 8, 1):
        print(f"  noalloc {cfg} T={T}", flush=True)
        x = W.make_x(bw.cfg, T, dev, seed=100 + T)
        assert block.workspace_size(T) <= lib.mlxr_moe_noalloc_scratch_size()
        want = block(x).clone()
        widx, ww = block.last_indices.clone(), block.last_weights.clone()
        got, idx, wts = _noalloc(pkg, block, x, T)
        torch.cuda.synchronize(dev)
        assert torch.equal(idx, widx) and torch.equal(wts, ww)
        assert torch.equal(got, want)
    del bw, block
    torch.cuda.empty_cache()


def test_noalloc_rejects_oversize_and_empty(pkg, dev):
    W = pkg.workloads
    bw = W.make_weights(W.CONFIGS["c2"], dev)
    block = bw.block()
    C = pkg._capi
    lib = C.lib()
    T = 4096
    assert block.workspace_size(T) > lib.mlxr_moe_noalloc_scratch_size()
    x = W.make_x(bw.cfg, 1, dev)
    rc = lib.mlxr_moe_block_forward_noalloc(ctypes.byref(block.descriptor()), x.data_ptr(), T,
                                            x.data_ptr(), None, None, None)
    assert rc == -1 and "scratch" in C.last_error() and "4096" in C.last_error()
    # T = 0 does nothing and succeeds
    assert lib.mlxr_moe_block_forward_noalloc(ctypes.byref(block.descriptor()), x.data_ptr(),
                                              0, x.data_ptr(), None, None, None) == 0


@pytest.mark.parametrize("T", [1, 64])
def test_noalloc_block_under_graph_capture(pkg, dev, T):
    """The no-allocation entry captured into a HIP graph (after the
    documented set-up call, mlxr_moe_noalloc_scratch_size, on this device)
    and replayed several times, with other eager block calls and
    synchronisations between the replays: every replay equals the eager
    call's output and routing bit for bit."""
    W = pkg.workloads
    bw = W.make_weights(W.CONFIGS["c2"], dev)
    block = bw.block()
    lib = pkg._capi.lib()
    assert lib.mlxr_moe_noalloc_scratch_size() == 32 * 1024 * 1024
    x = W.make_x(bw.cfg, T, dev, seed=200 + T)
    other = W.make_x(bw.cfg, 8, dev, seed=300 + T)
    want, widx, ww = _noalloc(pkg, block, x, T)
    want, widx, ww = want.clone(), widx.clone(), ww.clone()
    torch.cuda.synchronize(dev)
    print(f"  noalloc graph capture c2 T={T}", flush=True)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        # the static outputs of the captured call
        with torch.cuda.graph(g, stream=s):
            got, idx, wts = _noalloc(pkg, block, x, T)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize(dev)
    for rep in range(3):
        got.zero_()
        idx.zero_()
        # eager work between replays (its own scratch use and results)
        _noalloc(pkg, block, other, 8)
        torch.cuda.synchronize(dev)
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(idx, widx), rep
        assert torch.equal(wts, ww), rep
        assert torch.equal(got, want), rep
    del g, bw, block
    torch.cuda.empty_cache()
