"""Host logic of the device decode-state record (no GPU): the next token's
cache slot, visible key count and RoPE row, checked against a step-by-step
simulation of the reference's ring cache (KVCache::append / get_mask and
Qwen3Model::forward's start rule, example/qwen3/src/qwen3.cpp:70-126,
365-375) -- the rule the argmax kernels apply on the device."""
from __future__ import annotations

from ytensor_amd import ops


def _simulate(ring: int, max_pos: int, n: int):
    """KVCache bookkeeping for n single-token forwards: per step (start,
    write row, cur_len after the append, visible rows of the 1-row mask)."""
    cur_len = write_pos = total = 0
    out = []
    for _ in range(n):
        start = total if cur_len > 0 else 0
        if start + 1 > max_pos:
            start = cur_len
            if start + 1 > max_pos:
                start = 0
        row = write_pos
        write_pos = (write_pos + 1) % ring
        total += 1
        cur_len = min(cur_len + 1, ring)
        # get_mask(1) after the append: query logical position kv_len - 1
        if cur_len < ring:
            visible = [ki for ki in range(cur_len) if ki <= cur_len - 1]
        else:
            visible = [ki for ki in range(cur_len) if (ki - write_pos + ring) % ring <= cur_len - 1]
        out.append((start, row, cur_len, len(visible)))
    return out


def test_decode_state_matches_kvcache_simulation():
    for ring, max_pos in [(48, 48), (7, 7), (5, 9), (16, 4096)]:
        for total, (start, row, cur_len, nvis) in enumerate(_simulate(ring, max_pos, 3 * ring + 5)):
            slot, kv_len, rope = ops.decode_state_fields(total, ring, max_pos)
            assert (slot, kv_len, rope) == (row, cur_len, start), (ring, max_pos, total)
            assert nvis == kv_len  # every cached row is visible to the single query


def test_decode_state_record_layout():
    t = ops.decode_state(50, 48, 48, generated=3, history=100, device="cpu")
    assert t.dtype.is_floating_point is False and t.numel() == ops.ST_WORDS
    v = t.tolist()
    assert v[ops.ST_TOTAL] == 50 and v[ops.ST_SLOT] == 2 and v[ops.ST_KV_LEN] == 48 and v[ops.ST_ROPE_POS] == 0
    assert v[ops.ST_RING] == 48 and v[ops.ST_MAX_POS] == 48 and v[ops.ST_GENERATED] == 3 and v[ops.ST_HISTORY] == 100
    assert v[ops.ST_ERROR] == 0
