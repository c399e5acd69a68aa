"""Host-side checks of the module layer (no scan launches)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mlx_vision_mamba_amd import directions as dirs
from mlx_vision_mamba_amd import mamba_block as mb
from mlx_vision_mamba_amd import vision_mamba as vm
from mlx_vision_mamba_amd import vit
from oracle import scan_oracle as so
from oracle import torch_ref


@pytest.mark.parametrize("K,grid", [(2, None), (4, (14, 14)), (4, (3, 5)), (6, (4, 3, 5)),
                                    (8, (2, 3, 2, 4))])
def test_tables_match_oracle(K, grid):
    n = int(np.prod(grid)) if grid else 11
    table = dirs.seq_to_tok_table(K, n, grid)
    for k in range(K):
        axes, rev = so.direction_axis_order(K, k)
        np.testing.assert_array_equal(table[k].numpy(), so.seq_to_token(n, grid, axes, rev))
    inv = dirs.inverse_table(table)
    for k in range(K):
        np.testing.assert_array_equal(table[k][inv[k].long()].numpy(), np.arange(n))


def test_patch_embeds_equal_strided_convolution():
    torch.manual_seed(1)
    pe = vit.PatchEmbed(3, 8, 4).double()
    x = torch.randn(2, 16, 12, 3, dtype=torch.float64)
    ref = F.conv2d(x.permute(0, 3, 1, 2), pe.proj.weight, pe.proj.bias, stride=4)
    torch.testing.assert_close(pe(x), ref.flatten(2).transpose(1, 2))
    pe3 = vit.PatchEmbed3D(2, 8, 4).double()
    x3 = torch.randn(2, 8, 12, 4, 2, dtype=torch.float64)
    ref3 = F.conv3d(x3.permute(0, 4, 1, 2, 3), pe3.proj.weight, pe3.proj.bias, stride=4)
    torch.testing.assert_close(pe3(x3), ref3.flatten(2).transpose(1, 2))
    pe4 = vm.PatchEmbed4D(1, 8, 4, temporal_patch_size=2).double()
    x4 = torch.randn(2, 4, 8, 8, 4, 1, dtype=torch.float64)
    params = {"patch_embed.proj.weight": pe4.proj.weight, "patch_embed.proj.bias": pe4.proj.bias,
              "pos_embed": torch.zeros(1, 2 * 2 * 2 * 1, 8, dtype=torch.float64),
              "norm.weight": torch.ones(8, dtype=torch.float64),
              "norm.bias": torch.zeros(8, dtype=torch.float64)}
    ref4 = torch_ref.vision_mamba(params, x4, input_dim=4, patch_size=4, depth=0,
                                  grid_shape=(2, 2, 2, 1), d_state=16, d_conv=4,
                                  temporal_patch_size=2)
    got4 = F.layer_norm(pe4(x4), (8,), params["norm.weight"], params["norm.bias"], 1e-5)
    torch.testing.assert_close(got4, ref4)


def test_constructor_errors():
    with pytest.raises(ValueError):
        mb.MultiDirectionalMambaBlock(32, num_directions=3)
    with pytest.raises(ValueError):
        mb.MultiDirectionalMambaBlock(32, num_directions=4, grid_shape=None)
    with pytest.raises(ValueError):
        mb.MultiDirectionalMambaBlock(32, num_directions=6, grid_shape=(2, 2))
    with pytest.raises(ValueError):
        mb.MambaBlock(32, scan_mode="not_a_mode")
    with pytest.raises(ValueError):
        vm.VisionMamba(img_size=32, patch_size=16, embed_dim=16, depth=1, input_dim=5)


def test_scan_mode_passed_down():
    v = vm.VisionMamba(img_size=32, patch_size=16, embed_dim=16, depth=2, scan_mode="chunked")
    modes = {m.scan_mode for m in v.modules() if isinstance(m, mb.MambaBlock)}
    assert modes == {"chunked"}


def test_parameter_names_and_init():
    blk = mb.MambaBlock(d_model=48, d_state=16)
    names = dict(blk.named_parameters())
    assert names["in_proj.weight"].shape == (192, 48)
    assert names["conv1d.weight"].shape == (96, 1, 4)
    assert names["x_proj.weight"].shape == (3 + 32, 96)      # dt_rank = ceil(48/16) = 3
    assert names["dt_proj.weight"].shape == (96, 3)
    assert names["out_proj.weight"].shape == (48, 96)
    torch.testing.assert_close(-torch.exp(blk.A_log[0]), -torch.arange(1, 17, dtype=torch.float32))
    dt = F.softplus(blk.dt_proj.bias.detach())
    assert float(dt.min()) >= 1e-3 * (1 - 1e-5) and float(dt.max()) <= 1e-1 * (1 + 1e-5)


def test_direction_parameter_stacks_alias_and_rebuild():
    """The K direction blocks' parameters become slices of one (K, ...)
    buffer per kind with their values kept; a second call reuses the
    buffers; a dtype change (parameters moved one by one) rebuilds them."""
    torch.manual_seed(0)
    m = mb.MultiDirectionalMambaBlock(d_model=16, d_state=4, num_directions=4, grid_shape=(2, 3))
    blocks = list(m.mamba_blocks)
    before = {n: p.detach().clone() for n, p in m.named_parameters()}
    bufs = mb._direction_stacks(m, blocks)
    assert len(bufs) == len(mb.STACKED_PARAMS)
    for buf, name in zip(bufs, mb.STACKED_PARAMS):
        assert buf.shape[0] == 4
        for k, b in enumerate(blocks):
            p = mb._param(b, name)
            assert mb._is_slice_of(p, buf, k), name
            assert torch.equal(buf[k], before[f"mamba_blocks.{k}.{name}"])
    for n, p in m.named_parameters():
        assert torch.equal(p, before[n]), n
    assert mb._direction_stacks(m, blocks) is bufs
    # an in-place update through a parameter lands in the buffer
    with torch.no_grad():
        blocks[2].A_log.add_(1.0)
    assert torch.equal(bufs[mb.STACKED_PARAMS.index("A_log")][2], blocks[2].A_log)
    m.double()
    bufs2 = mb._direction_stacks(m, blocks)
    assert bufs2 is not bufs and bufs2[0].dtype == torch.float64
    assert all(mb._is_slice_of(mb._param(b, n), buf, k) for buf, n in zip(bufs2, mb.STACKED_PARAMS)
               for k, b in enumerate(blocks))


@pytest.mark.parametrize("K_used", [4, 2])
def test_direction_params_route_gradients_to_slices(K_used):
    """_DirectionParams returns the buffers (views, no copy) and hands each
    buffer's gradient to the parameters as slices: for a loss sum(w * buf)
    the gradient of block k's parameter is w[k]; with K_used < K (the
    two-direction fallback) only the first K_used blocks get gradients."""
    torch.manual_seed(1)
    m = mb.MultiDirectionalMambaBlock(d_model=16, d_state=4, num_directions=4, grid_shape=(2, 3))
    blocks = list(m.mamba_blocks)
    bufs = mb._direction_stacks(m, blocks)
    used = blocks[:K_used]
    outs = mb._DirectionParams.apply(len(bufs), *[b[:K_used] for b in bufs],
                                     *[mb._param(b, n) for n in mb.STACKED_PARAMS for b in used])
    ws = [torch.randn(o.shape, generator=torch.Generator().manual_seed(i)) for i, o in enumerate(outs)]
    for o, buf in zip(outs, bufs):
        assert o.data_ptr() == buf.data_ptr()
    sum((o * w).sum() for o, w in zip(outs, ws)).backward()
    for w, name in zip(ws, mb.STACKED_PARAMS):
        for k, b in enumerate(blocks):
            g = mb._param(b, name).grad
            if k < K_used:
                assert torch.equal(g, w[k]), (name, k)
            else:
                assert g is None, (name, k)


def test_permutation_check_on_host_tables():
    from mlx_vision_mamba_amd import scan
    t = dirs.seq_to_tok_table(4, 12, (3, 4))
    scan.check_permutation_table(t)
    assert t._mvm_perm_checked == (t.data_ptr(), t._version)
    bad = t.clone()
    bad[2, 0] = bad[2, 1]
    with pytest.raises(ValueError, match="permutation"):
        scan.check_permutation_table(bad)
    scan.check_permutation_table(torch.zeros(3, 0, dtype=torch.int32))


def test_host_table_is_checked_on_the_callers_tensor():
    """selective_scan_directions checks a host-memory table before copying
    it to the device, so the check's stamp sticks to the tensor the caller
    keeps and is not repeated for every fresh device copy (the call itself
    then stops at the CPU tensors: there is no CPU fallback)."""
    from mlx_vision_mamba_amd import scan
    K, L, D, N = 2, 6, 8, 4
    t = dirs.seq_to_tok_table(K, L, None)
    u = torch.randn(1, L, K, D)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        scan.selective_scan_directions(u, u.abs(), -torch.ones(K, D, N), torch.randn(1, L, K, N),
                                       torch.randn(1, L, K, N), torch.ones(K, D), seq_to_tok=t)
    assert t._mvm_perm_checked == (t.data_ptr(), t._version)


def test_replaced_scan_fn_is_detected():
    blk = mb.MambaBlock(16, scan_mode="chunked")
    assert not mb._custom_scan(blk)
    blk._scan_fn = lambda *a: a[0]
    assert mb._custom_scan(blk)
