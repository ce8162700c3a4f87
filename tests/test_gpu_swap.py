"""GPU: KV snapshot / restore (gg_kv_snapshot, gg_kv_restore), the swap path of the
reference's runner (internal/backend/cuda/swap_bridge.go:53-153). Blocks snapshotted to
pinned host memory and restored into other block ids must carry every layer's K and V
tiles (and PER_BLOCK scales) bit for bit, and attention over the moved blocks must equal
attention over the originals."""
import math

import numpy as np
import pytest
import torch

from gollmgo_amd._lib import DType
from gollmgo_amd.verify import KVCache
from helpers import say

pytestmark = pytest.mark.gpu

DTYPES = {"f32": DType.F32, "bf16": DType.BF16, "fp8": DType.FP8_E4M3, "int8": DType.INT8}
EB = {"f32": 4, "bf16": 2, "fp8": 1, "int8": 1}


def _tiles(kv, layer, H, bs, D, dt):
    """Per-block logical K and V tiles of one layer: [blocks][H][tile bytes] each."""
    tile = bs * D * EB[dt]
    k = kv.k_pool(layer).cpu().numpy().reshape(-1, H, tile)
    v = kv.v_pool(layer).cpu().numpy().reshape(-1, H, tile)
    return k, v


@pytest.mark.parametrize("dt,D", [("fp8", 128), ("int8", 128), ("bf16", 128), ("f32", 64)])
def test_snapshot_restore_moves_blocks(gpu, dt, D):
    say(f"kv swap dt={dt} D={D}")
    L, nb, H, bs = 3, 48, 4, 16
    kv = KVCache(L, nb, bs, H, D, DTYPES[dt])
    try:
        g = torch.Generator(device="cuda").manual_seed(5)
        if dt == "fp8":
            for layer in range(L):
                kv.set_head_scales(layer, [0.01 * (layer + 1)] * H, [0.02 * (layer + 1)] * H)
        slots = torch.arange(nb * bs, device="cuda", dtype=torch.int32)
        for layer in range(L):
            kv.append(layer, torch.randn(nb * bs, H, D, device="cuda", dtype=torch.bfloat16, generator=g),
                      torch.randn(nb * bs, H, D, device="cuda", dtype=torch.bfloat16, generator=g), slots)
        torch.cuda.synchronize()
        rng = np.random.default_rng(3)
        perm = rng.permutation(nb)
        src, dst = perm[:10].astype(np.int32), perm[10:20].astype(np.int32)
        before = [_tiles(kv, layer, H, bs, D, dt) for layer in range(L)]
        has_scales = dt in ("fp8", "int8")
        scales_before = [tuple(t.cpu().numpy().copy() for t in kv.scales(layer)) if has_scales else None
                         for layer in range(L)]
        nbytes = kv.snapshot_bytes(len(src))
        host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        staging, _ = kv.snapshot(torch.from_numpy(src).cuda(), host=host)
        torch.cuda.synchronize()
        host_copy = host.clone()
        staging.zero_()  # the restore must come from the host copy
        kv.restore(torch.from_numpy(dst).cuda(), staging, host=host_copy.pin_memory())
        torch.cuda.synchronize()
        for layer in range(L):
            k0, v0 = before[layer]
            k1, v1 = _tiles(kv, layer, H, bs, D, dt)
            np.testing.assert_array_equal(k1[dst], k0[src])
            np.testing.assert_array_equal(v1[dst], v0[src])
            untouched = np.setdiff1d(np.arange(nb), dst)
            np.testing.assert_array_equal(k1[untouched], k0[untouched])
            np.testing.assert_array_equal(v1[untouched], v0[untouched])
            if not has_scales:
                continue
            ks, vs = (t.cpu().numpy() for t in kv.scales(layer))
            if dt == "int8":  # PER_BLOCK scales travel with their blocks
                np.testing.assert_array_equal(ks[dst], scales_before[layer][0][src])
                np.testing.assert_array_equal(vs[dst], scales_before[layer][1][src])
            else:  # PER_HEAD scales stay with the layer
                np.testing.assert_array_equal(ks, scales_before[layer][0])
                np.testing.assert_array_equal(vs, scales_before[layer][1])
    finally:
        kv.close()


def test_attention_over_restored_blocks(gpu):
    """A sequence whose blocks were swapped out and restored elsewhere attends exactly as
    before (block table rewritten to the new ids); ids outside the pool give zero records on
    snapshot and are skipped on restore."""
    say("kv swap: attention over restored blocks")
    L, nb, H, bs, D, R, Hq = 2, 64, 8, 16, 128, 6, 32
    kv = KVCache(L, nb, bs, H, D, DType.FP8_E4M3)
    try:
        g = torch.Generator(device="cuda").manual_seed(9)
        for layer in range(L):
            kv.set_head_scales(layer, [4.5 / 448] * H, [4.5 / 448] * H)
            kv.append(layer, torch.randn(nb * bs, H, D, device="cuda", dtype=torch.bfloat16, generator=g),
                      torch.randn(nb * bs, H, D, device="cuda", dtype=torch.bfloat16, generator=g),
                      torch.arange(nb * bs, device="cuda", dtype=torch.int32))
        src = np.arange(0, 20, dtype=np.int32)           # the sequence's blocks (300 keys)
        dst = np.arange(40, 60, dtype=np.int32)
        keys = torch.tensor([300], dtype=torch.int32, device="cuda")
        q = torch.randn(1, R, Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
        outs = []
        with_bad = np.concatenate([src, [nb + 5]]).astype(np.int32)  # one id outside the pool
        staging, _ = kv.snapshot(torch.from_numpy(with_bad).cuda())
        rec = kv.snapshot_bytes(1) // L
        assert not staging[len(src) * L * rec:(len(src) + 1) * L * rec].any()  # zero record
        kv.restore(torch.from_numpy(np.concatenate([dst, [-1]]).astype(np.int32)).cuda(), staging)
        for ids in (src, dst):
            bt = torch.from_numpy(ids[None, :]).cuda()
            for layer in range(L):
                o = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
                kv.attention(layer, q, o, keys, bt, 1 / math.sqrt(D))
                outs.append(o.cpu().numpy())
        torch.cuda.synchronize()
        for layer in range(L):
            np.testing.assert_array_equal(outs[layer], outs[L + layer])
    finally:
        kv.close()
