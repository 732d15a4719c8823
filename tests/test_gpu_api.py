"""Entry-point contracts on the GPU: the bound row table of the asynchronous step is independent of the
synchronous step and of speculative verification; a failing row of the asynchronous step returns token -1
and reports its error through bl_slot_status; speculative rows whose dynamic temperature can reach 0 are
rejected; slots that were never set up are rejected."""
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import bl_select as BL  # noqa: E402

V, SEED = 151936, 2


def c2_params(r):
    return BL.Params(temperature=[0.0, 0.7, 1.0][r % 3], top_k=[0, 20, 64][r // 3], top_p=[1.0, 0.9][r % 2],
                     frequency_penalty=0.5, presence_penalty=0.3, logprobs=1, n_probs=10)


def reset_c2(ctx, slot, r):
    reply = BL.workload_ids(1, 2, SEED, r, 4096, V)
    ctx.slot_reset(slot, c2_params(r), BL.seed_rng(SEED + r), history=reply, reply=reply,
                   bias=BL.workload_bias(2, SEED, r, 300, V, -100.0, 100.0))


def test_bound_rows_survive_sync_steps_and_spec_verify_on_other_slots():
    """bind_rows(slots 0-3), then a synchronous step and a speculative verification on slots 4-7, then the
    asynchronous step: it samples and commits slots 0-3 exactly as a context that only stepped them."""
    dev = torch.device("cuda:0")
    n, steps = 4, 3
    pool = torch.empty((steps, 2 * n * V), dtype=torch.float32, device=dev)
    ref = BL.Context(V, n, n)
    for r in range(n):
        reset_c2(ref, r, r)
    for t in range(steps):
        ref.synth_logits(pool[t].data_ptr(), V, 2, SEED, t, 2 * n, V)
    want = [ref.sample_step(list(range(n)), pool[t].data_ptr(), V, top_stride=10)[:2] for t in range(steps)]
    ref.close()

    ctx = BL.Context(V, 2 * n, 2 * n)
    for r in range(2 * n):
        reset_c2(ctx, r, r)
    ctx.bind_rows(list(range(n)))
    tok = torch.zeros(n, dtype=torch.int32, device=dev)
    lp = torch.zeros(n, dtype=torch.float32, device=dev)
    ti = torch.zeros(n * 10, dtype=torch.int32, device=dev)
    tl = torch.zeros(n * 10, dtype=torch.float32, device=dev)
    other = list(range(n, 2 * n))
    for t in range(steps):
        other_rows = pool[t].data_ptr() + 4 * n * V  # rows n..2n-1 of this step's logits
        ctx.sample_step(other, other_rows, V, top_stride=10)
        ctx.spec_verify(other[:2], 1, other_rows, V, [7, 11])
        ctx.sample_step_async(n, pool[t].data_ptr(), V, tok.data_ptr(), lp.data_ptr(), ti.data_ptr(), tl.data_ptr(), 10)
        ctx.sync()
        assert tok.cpu().tolist() == want[t][0], f"step {t}"
        assert lp.cpu().tolist() == pytest.approx(want[t][1], rel=1e-6)
    ctx.close()


def test_async_failure_gives_token_minus_one_and_slot_status():
    """A full-vocabulary draw on a row of equal logits lands on a tie of V values, past the device's heap
    simulation (BL_ETIE at the step): through the asynchronous step its token is -1, nothing is committed,
    bl_slot_status reports the error once, and the other rows of the step are unaffected."""
    dev = torch.device("cuda:0")
    ctx = BL.Context(V, 2, 2)
    reset_c2(ctx, 0, 1)
    ctx.slot_reset(1, BL.Params(temperature=0.8, top_k=0), BL.seed_rng(9))
    logits = torch.empty(2 * V, dtype=torch.float32, device=dev)
    ctx.synth_logits(logits.data_ptr(), V, 2, SEED, 0, 2, V)
    logits[V:].zero_()
    rng_before = ctx.slot_rng(1)
    ctx.bind_rows([0, 1])
    tok = torch.zeros(2, dtype=torch.int32, device=dev)
    lp = torch.zeros(2, dtype=torch.float32, device=dev)
    ctx.sample_step_async(2, logits.data_ptr(), V, tok.data_ptr(), lp.data_ptr())
    ctx.sync()
    got = tok.cpu().tolist()
    assert got[1] == -1 and got[0] >= 0
    with pytest.raises(BL.BLError) as e:
        ctx.slot_status(1)
    assert e.value.code == BL.BL_ETIE
    ctx.slot_status(1)  # cleared by the first call
    ctx.slot_status(0)
    assert ctx.slot_rng(1) == rng_before  # nothing committed
    ctx.close()


def test_spec_rows_with_dynatemp_reaching_zero_are_rejected():
    ctx = BL.Context(V, 1, 3)
    ctx.slot_reset(0, BL.Params(temperature=0.5, dynatemp_range=0.6), BL.seed_rng(3))
    rows = torch.empty(3 * V, dtype=torch.float32, device="cuda:0")
    ctx.synth_logits(rows.data_ptr(), V, 5, 5, 0, 3, V)
    with pytest.raises(BL.BLError) as e:
        ctx.spec_verify([0], 2, rows.data_ptr(), V, [1, 2])
    assert e.value.code == BL.BL_EUNSUPPORTED
    ctx.slot_reset(0, BL.Params(temperature=0.5, dynatemp_range=0.4), BL.seed_rng(3))
    ctx.spec_verify([0], 2, rows.data_ptr(), V, [1, 2])  # tmin = 0.1 > 0: every row draws
    ctx.close()


def test_unready_slot_is_rejected():
    ctx = BL.Context(V, 2, 2)
    for call in (lambda: ctx.commit(1, [5]), lambda: ctx.slot_rng(1), lambda: ctx.slot_status(1)):
        with pytest.raises(BL.BLError) as e:
            call()
        assert e.value.code == BL.BL_EPARAM
    ctx.close()
