"""The host block-manager mirror against the reference's block_table_test.go cases."""
import pytest

from gollmgo_amd.blocks import BlockPool, BlockTable, OutOfBlocks


def test_block_table_reference_cases(golden):
    for c in golden["block_table"]:
        pool = BlockPool(c["pool"], c["bs"])
        bt = BlockTable(pool)
        bt.append_n(c["append"])
        if "free_after_append" in c:
            assert pool.num_free() == c["free_after_append"]
            bt.free()
            assert pool.num_free() == c["free_after_free"]
            assert bt.num_tokens == 0
            continue
        if c.get("then_append_fails"):
            with pytest.raises(OutOfBlocks):
                bt.append()
            continue
        if "truncate" in c:
            bt.truncate(c["truncate"])
        if "num_tokens" in c:
            assert bt.num_tokens == c["num_tokens"]
        if "num_blocks" in c:
            assert len(bt.blocks) == c["num_blocks"]
        if "free" in c:
            assert pool.num_free() == c["free"]


def test_slot_mapping_layout():
    pool = BlockPool(100, 4)
    bt = BlockTable(pool)
    bt.append_n(6)
    b0, b1 = bt.blocks
    assert bt.slot_mapping() == [b0 * 4 + i for i in range(4)] + [b1 * 4 + i for i in range(2)]


def test_shared_prefix_refcounts_and_appends():
    pool = BlockPool(20, 4)
    a = BlockTable(pool)
    a.append_n(8)
    b = BlockTable(pool)
    b.attach_shared(a.blocks[:2])
    assert all(pool.refcounts[x] == 2 for x in a.blocks[:2])
    slot = b.append()
    assert slot // 4 not in a.blocks  # appends never land in a shared block
    b.free()
    assert all(pool.refcounts[x] == 1 for x in a.blocks[:2])
