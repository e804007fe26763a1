"""ekv_dsa_decode_prologue_topk_merged against the two calls it stands for:
ekv_dsa_decode_prologue, then ekv_indexer_topk_merged of its outputs.

When the top-k runs as one launch the prologue is folded into it (each
workgroup prepares and quantizes its row's q itself; one workgroup per row
appends the new K and latent rows and writes the prologue's outputs).  Every
output must be the bytes of the two calls: both caches, the windowed
lengths, the q codes, the folded weights, the digit planes, the top-k rows
and the merged rows, and the fused path's counters left zero.  Cases: the
12-wave and the 4-wave kernels, with and without the indexer prep, bf16 and
fp32 head weights, tie-heavy rows (+4 sigma spikes), rows with no more keys
than k, rows with no keys, two rows per sequence, and the two-call fallback
(window 0, and 200 rows of one sequence: a chunk whose later rows score
the keys it appends)."""

import pytest
import torch

pytestmark = pytest.mark.gpu

WINDOW = 128

# (label, contexts, rows per sequence, indexer prep, spike kind, fp32 weights, window)
CASES = [
    ("12w_prep_sigma4", [300, 2176, 2177, 5000, 33000, 70000], 1, True, "sigma4", False, WINDOW),
    ("12w_two_rows_fp32w", [100, 3000, 9000, 40000], 2, False, "random_row", True, WINDOW),
    ("4w_prep", [2300] * 300, 1, True, "random_row", False, WINDOW),
    ("fallback_window0", [3000, 9000], 1, True, "random_row", False, 0),
    ("fallback_chunk_rows", [3000, 5000], 200, True, "random_row", False, WINDOW),
]


def _run(st, prep, weights, window, folded: bool, max_new_rows: int = 1):
    from ernie_kv import ops

    dev = st["kcache"].device
    B = st["B"]
    kc, lc = st["kcache"].clone(), st["latent"].clone()
    lengths = torch.full((B,), -7, dtype=torch.int32, device=dev)
    topk = torch.full((B, 2048), -9, dtype=torch.int32, device=dev)
    merged = torch.full((B, 2048 + WINDOW), -9, dtype=torch.int32, device=dev)
    ws = ops.indexer_topk_workspace(B, st["ctx"], dev)
    if folded:
        q8, wf, dg = ops.dsa_decode_prologue_topk_merged(
            st["k_new"], kc, st["latent_new"], lc, st["slots"], st["q_idx"], weights, st["positions"], window,
            lengths, st["block_table"], st["req_ids"], st["ctx"], topk, ws, merged, merged_slots=True, prep=prep,
            max_new_rows=max_new_rows)
    else:
        q8, wf, dg = ops.dsa_decode_prologue(st["k_new"], kc, st["latent_new"], lc, st["slots"], st["q_idx"],
                                             weights, st["positions"], window, lengths, prep=prep)
        ops.indexer_topk_merged(q8, dg, wf, kc, st["block_table"], st["req_ids"], lengths, st["ctx"], topk, ws,
                                merged=merged, positions=st["positions"], window=window, merged_slots=True)
    torch.cuda.synchronize()
    counters = ws[: ops.indexer_topk_counter_bytes()]
    return dict(kcache=kc, latent=lc, lengths=lengths, q8=q8, w=wf, digits=dg, topk=topk, merged=merged,
                counters_zero=bool((counters[256:] == 0).all()))


@pytest.mark.parametrize("label,ctxs,R,prep_on,spikes,fp32_w,window", CASES, ids=[c[0] for c in CASES])
def test_folded_prologue_matches_two_calls(dev, label, ctxs, R, prep_on, spikes, fp32_w, window):
    import bench
    from ernie_kv import ops

    print(f"[folded {label}] build", flush=True)
    st = bench.build_dsa_decode(torch, ops, ctxs, 5, rows_per_seq=R, spikes=spikes)
    prep = (st["ln_w"], st["ln_b"], 1e-6, st["rope"]) if prep_on else None
    weights = st["w_idx"].float().contiguous() if fp32_w else st["w_idx"]
    folds = ops.dsa_decode_prologue_folds(st["B"], st["ctx"])
    assert folds, f"{label}: the plan should run as one launch"
    print(f"[folded {label}] two calls", flush=True)
    ref = _run(st, prep, weights, window, folded=False)
    print(f"[folded {label}] one call", flush=True)
    got = _run(st, prep, weights, window, folded=True, max_new_rows=R)
    for key in ("kcache", "latent", "lengths", "q8", "w", "digits", "topk", "merged"):
        a, b = ref[key], got[key]
        if a.dtype == torch.float32:
            a, b = a.view(torch.int32), b.view(torch.int32)
        bad = (a != b).nonzero()
        assert bad.numel() == 0, f"{label}: {key} differs at {bad[:8].tolist()} ({bad.shape[0]} entries)"
    assert ref["counters_zero"] and got["counters_zero"]


def test_folded_prologue_when_every_wait_gives_up(dev):
    """With the waits' poll limit at 0 every row's workgroups stop waiting for
    one another (each row then selects alone, exactly): the folded
    prologue's outputs and appends, written by the row's first workgroup to
    arrive before it waits, must still be the two calls' bytes."""
    import bench
    from ernie_kv import ops

    st = bench.build_dsa_decode(torch, ops, [5000, 20000, 2177, 9000], 7, spikes="random_row")
    prep = (st["ln_w"], st["ln_b"], 1e-6, st["rope"])
    ref = _run(st, prep, st["w_idx"], WINDOW, folded=False)
    prev = ops.indexer_set_spin_limit(0)
    try:
        got = _run(st, prep, st["w_idx"], WINDOW, folded=True)
    finally:
        ops.indexer_set_spin_limit(prev)
    for key in ("kcache", "latent", "lengths", "q8", "w", "digits", "topk", "merged"):
        a, b = ref[key], got[key]
        if a.dtype == torch.float32:
            a, b = a.view(torch.int32), b.view(torch.int32)
        assert torch.equal(a, b), key
    assert got["counters_zero"]
