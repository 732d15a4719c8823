"""HIP-graph capture of the asynchronous step: replays (with eager work and synchronisations between
them) give the same tokens and logprobs as the synchronous eager step on an identical context."""
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import bl_select as BL  # noqa: E402

V, B, SEED = 151936, 8, 2


def make_ctx():
    ctx = BL.Context(V, B, B)
    for r in range(B):
        p = BL.Params(temperature=[0.0, 0.7, 1.0][r % 3], top_k=[0, 20, 64][r // 3], top_p=[1.0, 0.9][r % 2],
                      frequency_penalty=0.5, presence_penalty=0.3, logprobs=1, n_probs=10)
        reply = BL.workload_ids(1, 2, SEED, r, 4096, V)
        ctx.slot_reset(r, p, BL.seed_rng(SEED + r), history=reply, reply=reply,
                       bias=BL.workload_bias(2, SEED, r, 300, V, -100.0, 100.0))
    return ctx


def test_graph_replay_matches_eager():
    dev = torch.device("cuda:0")
    steps = 6
    pool = torch.empty((steps, B * V), dtype=torch.float32, device=dev)
    eager = make_ctx()
    for t in range(steps):
        eager.synth_logits(pool[t].data_ptr(), V, 2, SEED, t, B, V)
    want = [eager.sample_step(list(range(B)), pool[t].data_ptr(), V, top_stride=10)[:2] for t in range(steps)]
    eager.close()

    ctx = make_ctx()
    ctx.bind_rows(list(range(B)))
    s = torch.cuda.Stream()
    ctx.set_stream(s.cuda_stream)
    tok = torch.zeros(B, dtype=torch.int32, device=dev)
    lp = torch.zeros(B, dtype=torch.float32, device=dev)
    ti = torch.zeros(B * 10, dtype=torch.int32, device=dev)
    tl = torch.zeros(B * 10, dtype=torch.float32, device=dev)
    graphs = []
    for t in range(steps):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            ctx.sample_step_async(B, pool[t].data_ptr(), V, tok.data_ptr(), lp.data_ptr(), ti.data_ptr(),
                                  tl.data_ptr(), 10)
        graphs.append(g)
    torch.cuda.synchronize()
    for t in range(steps):
        junk = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
        with torch.cuda.stream(s):
            graphs[t].replay()
        torch.cuda.synchronize()
        assert tok.cpu().tolist() == want[t][0], f"step {t}"
        assert lp.cpu().tolist() == pytest.approx(want[t][1], rel=1e-6)
        del junk
    ctx.close()


def test_library_step_graph_matches_eager():
    """bl_step_graph_create / bl_step_graph_launch: graphs captured by the library on its own stream,
    each replayed twice around eager work, the second replay continuing the slots' state like a second
    eager step."""
    dev = torch.device("cuda:0")
    steps = 4
    pool = torch.empty((steps, B * V), dtype=torch.float32, device=dev)
    eager = make_ctx()
    for t in range(steps):
        eager.synth_logits(pool[t].data_ptr(), V, 2, SEED, t, B, V)
    want = []
    for t in range(steps):
        for _ in range(2):
            want.append(eager.sample_step(list(range(B)), pool[t].data_ptr(), V, top_stride=10)[:3])
    eager.close()

    ctx = make_ctx()
    ctx.bind_rows(list(range(B)))
    tok = torch.zeros(B, dtype=torch.int32, device=dev)
    lp = torch.zeros(B, dtype=torch.float32, device=dev)
    ti = torch.zeros(B * 10, dtype=torch.int32, device=dev)
    tl = torch.zeros(B * 10, dtype=torch.float32, device=dev)
    graphs = [ctx.step_graph(B, pool[t].data_ptr(), V, tok.data_ptr(), lp.data_ptr(), ti.data_ptr(), tl.data_ptr(), 10)
              for t in range(steps)]
    try:
        i = 0
        for t in range(steps):
            for _ in range(2):
                junk = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
                ctx.graph_launch(graphs[t])
                ctx.sync()
                torch.cuda.synchronize()
                assert tok.cpu().tolist() == want[i][0], f"replay {i}"
                assert lp.cpu().tolist() == pytest.approx(want[i][1], rel=1e-6)
                assert ti.cpu().tolist() == [x for row in want[i][2] for x in row], f"replay {i}"
                del junk
                i += 1
    finally:
        for g in graphs:
            BL.Context.graph_destroy(g)
        ctx.close()
