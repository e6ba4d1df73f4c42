"""The engine's contract with the GPU layer (src/engine.rs:190-241), through the C ABI.

Engine::synth_batch plans length-bucketed microbatches and, when forward_batch returns an error,
splits the batch in two and retries the halves (a stack, first half first), down to single items
whose error is that item's result.  The library must therefore (1) report device-memory exhaustion
as an error (KK_ERR_OOM), never an abort, and (2) give every item the same result whatever batch it
ends up in, in input order.  The OOM is forced from the host with the library's test hook
KOKORO_HIP_TEST_OOM_ABOVE=k (batches of more than k items fail as an allocation would).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

KK_ERR_OOM = -3


def synth_batch(ctx, items, max_batch, call=None):
    """Engine::synth_batch's retry loop (src/engine.rs:213-239) over forward_decoder_batch (or
    `call`): returns per-item results or the KKError of a single item, and the sizes of the calls
    made."""
    from kokoro_hip import api
    results = [None] * len(items)
    # plan_batches (src/engine.rs:165-183) with a fixed cap: consecutive chunks of max_batch
    plan = [list(range(i, min(i + max_batch, len(items)))) for i in range(0, len(items), max_batch)]
    stack = list(reversed(plan))
    calls = []
    while stack:
        batch = stack.pop()
        calls.append(len(batch))
        try:
            outs = (call or ctx.forward_decoder_batch)([items[k] for k in batch])
        except api.KKError as e:
            if len(batch) > 1:
                mid = len(batch) // 2
                stack.append(batch[mid:])
                stack.append(batch[:mid])
            else:
                results[batch[0]] = e
            continue
        for k, o in zip(batch, outs):
            results[k] = o
    return results, calls


def test_halving_on_oom_keeps_order_and_bits(gpu_ctx, monkeypatch):
    from kokoro_hip import workloads
    items = workloads.small_items(81, [13, 4, 21, 9, 2, 17, 6])
    full = gpu_ctx.forward_decoder_batch(items)
    monkeypatch.setenv("KOKORO_HIP_TEST_OOM_ABOVE", "2")
    res, calls = synth_batch(gpu_ctx, items, max_batch=8)
    print("  calls:", calls, flush=True)
    # 7 fails -> [0..2] fails -> [0] ok, [1, 2] ok; [3..6] fails -> [3, 4] ok, [5, 6] ok
    assert calls == [7, 3, 1, 2, 4, 2, 2]
    for k, (a, b) in enumerate(zip(full, res)):
        assert isinstance(b, np.ndarray) and np.array_equal(a, b), f"item {k}"


def test_single_item_oom_is_that_items_error(gpu_ctx, monkeypatch):
    from kokoro_hip import api, workloads
    items = workloads.small_items(82, [5, 8])
    monkeypatch.setenv("KOKORO_HIP_TEST_OOM_ABOVE", "0")
    res, calls = synth_batch(gpu_ctx, items, max_batch=8)
    assert calls == [2, 1, 1]
    for r in res:
        assert isinstance(r, api.KKError) and r.code == KK_ERR_OOM
    # the context stays usable once the pressure is gone
    monkeypatch.delenv("KOKORO_HIP_TEST_OOM_ABOVE")
    again = gpu_ctx.forward_decoder_batch(items)
    with api.Plan.decoder(gpu_ctx, items) as plan:
        plan.run()
        ref = plan.fetch()
    for a, b in zip(ref, again):
        assert np.array_equal(a, b)


def test_ids_level_halving_on_oom(monkeypatch):
    """The same loop over the ids-level entry (kk_forward_batch, the call Engine::synth_batch makes
    on the reference): every item's audio and durations bit-identical to the unsplit batch, in
    input order; a single item's OOM is that item's error."""
    from kokoro_hip import api, model_spec, workloads
    ctx = api.Context(0)
    try:
        ctx.upload_model(model_spec.random_model_weights(seed=0))
        items = workloads.small_ids_items(85, [14, 3, 30, 8, 22])
        full = ctx.forward_batch(items)
        monkeypatch.setenv("KOKORO_HIP_TEST_OOM_ABOVE", "2")
        res, calls = synth_batch(ctx, items, max_batch=8, call=ctx.forward_batch)
        print("  calls:", calls, flush=True)
        # 5 fails -> [0, 1] ok; [2, 3, 4] fails -> [2] ok, [3, 4] ok
        assert calls == [5, 2, 3, 1, 2]
        for k, ((a, d), r) in enumerate(zip(full, res)):
            assert isinstance(r, tuple) and np.array_equal(a, r[0]) and np.array_equal(d, r[1]), f"item {k}"
        monkeypatch.setenv("KOKORO_HIP_TEST_OOM_ABOVE", "0")
        res, calls = synth_batch(ctx, items[:2], max_batch=8, call=ctx.forward_batch)
        assert calls == [2, 1, 1] and all(isinstance(r, api.KKError) and r.code == KK_ERR_OOM for r in res)
    finally:
        ctx.close()
