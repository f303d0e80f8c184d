"""Host-side argument checks of the Python mirrors: shapes, dtypes and
devices are rejected before any pointer reaches the C ABI (no GPU needed:
every case here fails before a kernel could run)."""
import pytest
import torch


def _tiny_block(pkg, d=128, E=4, f=64, K=2):
    nn = pkg.nn
    q = lambda out, inp: nn.QuantizedSwitchLinear(  # noqa: E731
        torch.zeros((E, out, inp // 8), dtype=torch.int32),
        torch.zeros((E, out, inp // 64), dtype=torch.bfloat16),
        torch.zeros((E, out, inp // 64), dtype=torch.bfloat16), 64, 4)
    mlp = nn.SplitSwitchFfn(q(f, d), q(f, d), q(d, f))
    return nn.Qwen35MoeBlock(torch.zeros((E, d)), mlp, K)


@pytest.mark.parametrize("xs,idx", [((), (5, 2)), ((5, 1), (5, 2)), ((1,), (5, 2)),
                                    ((5, 2), (5, 2)), ((3, 1, 1), (3, 4, 2)),
                                    ((1, 5, 1), (5, 2)), ((3, 4, 1), (3, 4, 2))])
def test_x_batch_forms_accepted(pkg, xs, idx):
    pkg.ops._check_x_batch("gather_qmm", xs, idx)


@pytest.mark.parametrize("xs,idx", [((1, 3), (2, 3)), ((2,), (2, 3)), ((1, 2), (3, 2)),
                                    ((4, 1), (5, 2)), ((2, 5, 1), (5, 2))])
def test_x_batch_forms_rejected(pkg, xs, idx):
    """A leading singleton broadcast against a larger index axis (MLX would
    take x row b % 3; the kernels' b // (B / x_batch) would not)."""
    with pytest.raises(pkg.MlxrMoeError, match="batch shape"):
        pkg.ops._check_x_batch("gather_qmm", xs, idx)


def test_gather_qmm_rejects_broadcast_before_launch(pkg):
    x = torch.zeros((1, 3, 1, 64), dtype=torch.bfloat16)
    idx = torch.zeros((2, 3), dtype=torch.int32)
    with pytest.raises(pkg.MlxrMoeError, match="batch shape"):
        pkg.ops.gather_qmm(x, torch.zeros((4, 64, 8), dtype=torch.int32),
                           torch.zeros((4, 64, 1), dtype=torch.bfloat16),
                           torch.zeros((4, 64, 1), dtype=torch.bfloat16), None, idx)
    with pytest.raises(pkg.MlxrMoeError, match="batch shape"):
        pkg.ops.gather_mm(x, torch.zeros((4, 64, 64), dtype=torch.bfloat16), None, idx)


def test_block_rejects_wrong_x_before_launch(pkg):
    blk = _tiny_block(pkg)
    with pytest.raises(pkg.MlxrMoeError, match="must be torch.bfloat16"):
        blk.forward(torch.zeros((3, 128), dtype=torch.float32))
    with pytest.raises(pkg.MlxrMoeError, match="last dim must be 128"):
        blk.forward(torch.zeros((3, 64), dtype=torch.bfloat16))
    with pytest.raises(pkg.MlxrMoeError, match="ROCm device"):
        blk.forward(torch.zeros((3, 128), dtype=torch.bfloat16))
    norm = pkg.nn.RmsNorm(torch.ones(64))
    with pytest.raises(pkg.MlxrMoeError, match="norm weight must have 128"):
        blk.forward_residual(torch.zeros((3, 128), dtype=torch.bfloat16), norm)
    with pytest.raises(pkg.MlxrMoeError, match="must be torch.bfloat16"):
        blk.forward_residual(torch.zeros((3, 128), dtype=torch.float16), norm)
    with pytest.raises(pkg.MlxrMoeError, match="must be torch.bfloat16"):
        blk.switch_mlp.forward(torch.zeros((3, 128)), torch.zeros((3, 2), dtype=torch.int32))
    with pytest.raises(pkg.MlxrMoeError, match="must be torch.bfloat16"):
        pkg.nn.RmsNorm(torch.ones(128)).forward(torch.zeros((3, 128)))


def test_out_checks(pkg):
    chk = pkg.nn._check_out
    dev = torch.device("cpu")
    chk("b", torch.empty((3, 128)), 3, 128, torch.float32, dev)
    chk("b", torch.empty((1, 3, 128)), 3, 128, torch.float32, dev)
    with pytest.raises(pkg.MlxrMoeError, match="must be torch.float32"):
        chk("b", torch.empty((3, 128), dtype=torch.bfloat16), 3, 128, torch.float32, dev)
    with pytest.raises(pkg.MlxrMoeError, match=r"shape \(3, 128\)"):
        chk("b", torch.empty((2, 128)), 3, 128, torch.float32, dev)
    with pytest.raises(pkg.MlxrMoeError, match=r"shape \(3, 128\)"):
        chk("b", torch.empty((128, 3)), 3, 128, torch.float32, dev)
    with pytest.raises(pkg.MlxrMoeError, match="contiguous"):
        chk("b", torch.empty((128, 3)).t(), 3, 128, torch.float32, dev)
    with pytest.raises(pkg.MlxrMoeError, match="must be on"):
        chk("b", torch.empty((3, 128), device="meta"), 3, 128, torch.float32, dev)


def test_noalloc_refuses_oversize_on_host(pkg):
    """The no-alloc block forward refuses a T whose workspace exceeds the
    library's scratch array before touching the device (host pointers
    here are never dereferenced)."""
    import ctypes
    blk = _tiny_block(pkg)
    lib, C = pkg._capi.lib(), pkg._capi
    cap = lib.mlxr_moe_noalloc_scratch_size()
    T = 1
    while blk.workspace_size(T) <= cap:
        T *= 2
    x = torch.zeros(16, dtype=torch.bfloat16)
    rc = lib.mlxr_moe_block_forward_noalloc(ctypes.byref(blk.descriptor()), x.data_ptr(), T,
                                            x.data_ptr(), None, None, None)
    assert rc == -1 and "scratch" in C.last_error() and str(T) in C.last_error()
    assert lib.mlxr_moe_block_forward_noalloc(None, None, 1, None, None, None, None) == -1
    assert "null module" in C.last_error()


@pytest.mark.parametrize("key", ["c3", "c5"])
def test_zipf_fixture(pkg, key):
    """The committed Zipf routing fixture (tests/golden/zipf_routing.npz,
    written by make_zipf_routing.py): a finite bias per expert, and at
    every bench T row counts that sum to T*K, never exceed T (top-K picks an
    expert at most once per token) and follow the Zipf(1.1) order of the
    seeded permutation (the expert of rank 1 the fullest, the top decile
    of ranks holding most of the rows)."""
    import numpy as np
    W = pkg.workloads
    cfg = W.CONFIGS[key]
    b = W.zipf_bias(cfg, "cpu")
    assert tuple(b.shape) == (cfg.E,) and bool(torch.isfinite(b).all())
    with np.load(W.ZIPF_FIXTURE) as z:
        perm = z[f"{cfg.name}__perm"]
    assert sorted(perm.tolist()) == list(range(cfg.E))
    for T in cfg.tokens:
        rows = W.zipf_rows(cfg, T)
        assert rows is not None and rows.shape == (cfg.E,)
        assert int(rows.sum()) == T * cfg.K and int(rows.max()) <= T
        by_rank = rows[perm]
        assert by_rank[0] == rows.max()
        if T >= 512:
            top = by_rank[: cfg.E // 10].sum()
            assert top > 0.5 * T * cfg.K
