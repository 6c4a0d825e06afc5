"""The whole decode step (iam_model_*) against the oracle's model on a small
Mistral-shaped configuration: 2 layers, dim 4096 (32 heads x 128, 8 KV
heads), FFN 4096, vocabulary 512, 64 positions.

Bar: synthesized weights byte-identical to the oracle generator + bucketizer;
logits within 1 ulp of the oracle's at every step (default fp64
accumulation, both sides running free on their own intermediates); greedy
tokens identical to the oracle's; eager and graph-replayed steps give the
same bits; in fp32 accumulation the steps are still deterministic and the LM
head matches the oracle under teacher forcing."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=2, dim=4096, ffn_dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, vocab=512,
           max_ctx=64, rope_theta=10000.0, norm_eps=1e-5)
def tid_layer(L, k):
    return 1000 + 16 * L + k


@pytest.fixture(scope="module")
def model(iam, ctx):
    cfg = iam.ModelConfig(**CFG)
    m = iam.Model(ctx, cfg)
    m.synthesize(0)
    yield m
    m.close()


def OracleModel(O, m):
    return O.OracleModel(CFG, m.read_tensor)


def test_synthesized_weights_match_oracle(O, model):
    for L, w, k, shape in [(0, "wk", 1, (1024, 4096)), (1, "w2", 6, (4096, 4096))]:
        W = O.gen_f16(0, tid_layer(L, k), shape[0] * shape[1], 0.0, 0.02).reshape(shape)
        b, s, p = O.bucketize(W)
        assert np.array_equal(model.read_tensor(f"layer{L}.{w}.buckets", np.uint16), b.ravel())
        assert np.array_equal(model.read_tensor(f"layer{L}.{w}.stats", np.uint16), s.ravel())
        assert np.array_equal(model.read_tensor(f"layer{L}.{w}.probes", np.uint16), p)
        assert np.array_equal(model.read_tensor(f"layer{L}.{w}.stats3", np.uint16), s[:, 3])
    assert np.array_equal(model.read_tensor("layer1.ffn_gain", np.uint16), O.gen_f16(0, tid_layer(1, 8), 4096, 1.0, 0.01))
    assert np.array_equal(model.read_tensor("embed", np.uint16), O.gen_f16(0, 10, 512 * 4096, 0.0, 0.02))
    assert np.array_equal(model.read_tensor("final_gain", np.uint16), O.gen_f16(0, 11, 4096, 1.0, 0.01))


def ulps(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def lm_head_teacher_forced(O, model, effort):
    """Oracle final norm + LM head applied to the GPU's own final hidden state."""
    h = model.read_tensor("hidden", np.float32)
    hn = model.read_tensor("hidden_norm", np.float32)
    want = O.rmsnorm_gain(h, model.read_tensor("final_gain", np.uint16), CFG["norm_eps"])
    assert np.linalg.norm(hn - want) / np.linalg.norm(want) < 1e-6
    b = model.read_tensor("lm_head.buckets", np.uint16).reshape(CFG["dim"] * 16, CFG["vocab"] // 16)
    s = model.read_tensor("lm_head.stats", np.uint16).reshape(CFG["dim"] * 16, 4)
    p = model.read_tensor("lm_head.probes", np.uint16)
    y, cut, mask, S = O.bucketmul(hn, s, p, b, effort)
    return y


@pytest.mark.parametrize("effort", [0.25, 1.0])
def test_logits_match_oracle_every_step(O, ctx, model, effort):
    """Both models run free for 8 steps on the same tokens; the logits stay
    within 1 ulp of the oracle's at every step."""
    orc = OracleModel(O, model)
    model.reset_caches()
    dlog = ctx.empty(CFG["vocab"], np.float32)
    toks = O.gen_tokens(0, 99, 8, CFG["vocab"]).tolist()
    for pos, tok in enumerate(toks):
        model.forward(tok, pos, effort, dlog)
        lg = dlog.read()
        lo = orc.forward(tok, pos, effort)
        assert ulps(lg, lo).max() <= 1, pos
    dlog.free()


@pytest.mark.parametrize("effort", [0.25, 1.0])
def test_lm_head_teacher_forced_every_step(O, ctx, model, effort):
    """At every step the logits equal the oracle's final norm + LM head on the
    GPU's own hidden state (identical input, so the cutoff and the selected
    rows are the same and only fp32 summation order differs)."""
    model.reset_caches()
    prompt = O.gen_tokens(0, 97, 4, CFG["vocab"]).tolist()
    dlog = ctx.empty(CFG["vocab"], np.float32)
    seq = list(prompt)
    for pos in range(len(prompt) + 6):
        model.forward(seq[pos], pos, effort, dlog)
        lg = dlog.read()
        y = lm_head_teacher_forced(O, model, effort)
        assert np.linalg.norm(lg - y) / np.linalg.norm(y) < 1e-5, pos
        if pos >= len(prompt) - 1:
            seq.append(int(np.argmax(lg)))
    dlog.free()


def test_generate_graph_equals_eager_and_picks_argmax(O, ctx, model):
    """Greedy generation: graph-replayed steps (9 new steps: one graph of 8
    captured steps, then a one-step graph) give the eager steps' tokens, in
    both accumulation modes, and every picked token is the first maximum of
    the oracle LM head on the GPU's own hidden state."""
    prompt = O.gen_tokens(0, 98, 5, CFG["vocab"]).tolist()
    n_new = 10
    for mode in ("fp32", "fp64"):
        ctx.set_accumulation(mode)
        model.reset_caches()
        eager = model.generate(prompt, n_new, 0.25, use_graph=False).tolist()
        model.reset_caches()
        graph = model.generate(prompt, n_new, 0.25, use_graph=True).tolist()
        model.reset_caches()
        graph2 = model.generate(prompt, n_new, 0.25, use_graph=True).tolist()   # replays the captured step
        assert eager == graph == graph2, mode
    # replay the same sequence eagerly and check each pick against the oracle head
    model.reset_caches()
    dlog = ctx.empty(CFG["vocab"], np.float32)
    seq = prompt + eager
    for pos in range(len(prompt) + n_new - 1):
        model.forward(seq[pos], pos, 0.25, dlog)
        if pos >= len(prompt) - 1:
            y = lm_head_teacher_forced(O, model, 0.25)
            assert O.argmax(y) == seq[pos + 1], pos
    dlog.free()


def test_counting_off_gives_the_same_tokens(O, ctx, model):
    """Graph-replayed greedy decode with the walk counting switched off (the
    decode graph is re-captured) picks the same tokens, and the counters do
    not move."""
    prompt = O.gen_tokens(0, 96, 5, CFG["vocab"]).tolist()
    model.reset_caches()
    on = model.generate(prompt, 6, 0.25, use_graph=True).tolist()
    ctx.walk_counters(reset=True)
    ctx.set_walk_counting(False)
    try:
        model.reset_caches()
        off = model.generate(prompt, 6, 0.25, use_graph=True).tolist()
        assert ctx.walk_counters(reset=True) == (0, 0, 0)
    finally:
        ctx.set_walk_counting(True)
    assert off == on
    model.reset_caches()
    again = model.generate(prompt, 6, 0.25, use_graph=True).tolist()
    assert again == on
    assert ctx.walk_counters(reset=True)[2] > 0


def test_search_hint_counters(O, ctx, model):
    """Each walk of a decode step starts its cutoff search from the same
    matrix's cutoff of the previous step: at effort 0.25 (rank 1025) every
    group takes hints and nearly all hold (the first step after the reset
    has none); at effort 1.0 (rank 4096, within 64 of the end) none is
    taken.  Hits never exceed tries, and the tokens are those of an
    unhinted run (test_greedy_tokens_match_oracle, which checks them
    against the oracle, runs with hints too)."""
    prompt = O.gen_tokens(0, 97, 12, CFG["vocab"]).tolist()
    for effort, want in ((0.25, True), (1.0, False)):
        model.reset_caches()
        ctx.walk_counters(reset=True)
        model.generate(prompt, 4, effort, use_graph=True)
        for g in ("qkv", "o", "ffn13", "ffn2", "lm"):
            tries, hits = ctx.walk_group_hints(g)
            assert hits <= tries, (effort, g, tries, hits)
            if want:
                assert tries > 0 and hits >= 0.7 * tries, (effort, g, tries, hits)
            else:
                assert tries == 0, (effort, g, tries)
    ctx.walk_counters(reset=True)


@pytest.mark.parametrize("effort", [0.05, 1.0])
def test_skewed_embedding_logits_match_oracle(O, ctx, model, effort):
    """Skew stress: 1% of the hidden channels (41 of 4096) scaled 20x after
    the embedding gather.  The oracle takes the same scaled embedding row as
    its hidden input; logits within 1 ulp at every step, both running free."""
    rng = np.random.default_rng(11)
    scale = np.ones(CFG["dim"], np.float32)
    scale[rng.choice(CFG["dim"], CFG["dim"] // 100, replace=False)] = 20.0
    emb = O.f16_to_f32(model.read_tensor("embed", np.uint16)).reshape(CFG["vocab"], CFG["dim"])
    orc = OracleModel(O, model)
    model.reset_caches()
    model.set_embed_scale(scale)
    dlog = ctx.empty(CFG["vocab"], np.float32)
    try:
        for pos, tok in enumerate(O.gen_tokens(0, 93, 6, CFG["vocab"]).tolist()):
            model.forward(tok, pos, effort, dlog)
            lo = orc.forward(tok, pos, effort, hidden_in=emb[tok] * scale)
            assert ulps(dlog.read(), lo).max() <= 1, pos
    finally:
        model.set_embed_scale(None)
        dlog.free()


def test_greedy_tokens_match_oracle(O, model):
    """Greedy decode from a 5-token prompt: the GPU's 16 new tokens (graph
    replay) are the oracle's."""
    orc = OracleModel(O, model)
    prompt = O.gen_tokens(0, 95, 5, CFG["vocab"]).tolist()
    n_new = 16
    model.reset_caches()
    gpu = model.generate(prompt, n_new, 0.25, use_graph=True).tolist()
    seq = list(prompt)
    for pos in range(len(prompt) + n_new - 1):
        lo = orc.forward(seq[pos], pos, 0.25)
        if pos >= len(prompt) - 1:
            seq.append(O.argmax(lo))
    assert gpu == seq[len(prompt):]


def test_model_rejects_bad_config(iam, ctx):
    bad = dict(CFG)
    bad["dim"] = 2048
    bad["n_heads"] = 16
    with pytest.raises(iam.IamError):
        iam.Model(ctx, iam.ModelConfig(**bad))


def test_block_selection_model_logits_and_tokens(O, ctx, model):
    """The decode step with block-structured selection (blocks of 8 inputs
    below effort 0.5), run at effort 0.25: logits within 1 ulp of the oracle
    model with the same selection at every step, greedy tokens identical,
    and different from the per-row selection's logits."""
    orc = OracleModel(O, model)
    prompt = [5, 77, 130]
    ctx.set_selection_block(8, 0.5)
    O.set_selection_block(8, 0.5)
    try:
        toks = model.generate(np.array(prompt, np.int32), 4, 0.25, use_graph=True)
        seq = list(prompt)
        for pos in range(len(prompt) + 3):
            lo = orc.forward(seq[pos], pos, 0.25)
            if pos >= len(prompt) - 1:
                seq.append(O.argmax(lo))
        assert list(toks) == seq[len(prompt):]
        gl = ctx.empty(CFG["vocab"], np.float32)
        model.forward(seq[2], 2, 0.25, gl)
        g = gl.read()
        want = orc.forward(seq[2], 2, 0.25)
        assert ulps(g, want).max() <= 1
        O.set_selection_block(1)
        fine = orc.forward(seq[2], 2, 0.25)
        assert not np.array_equal(fine, want)
        gl.free()
    finally:
        ctx.set_selection_block(1)
        O.set_selection_block(1)


def test_model_refuses_steps_past_the_kv_capacity(iam, ctx, model):
    """The host keeps the position of the next step: a decode, device step or
    generate that would write K/V past max_ctx, or a position beyond
    max_ctx (max_ctx itself is the full cache), fails with IAM_E_INVALID
    before anything is launched; the steps up to the last slot run."""
    cap = CFG["max_ctx"]
    model.generate(np.arange(4, dtype=np.int32), 1, 0.25, use_graph=False)   # next step at position 4
    model.decode(cap - 4 - 1, 0.25, use_graph=False)                         # positions 4 .. cap - 2
    model.decode(1, 0.25, use_graph=True)                                    # cap - 1, the last slot
    ctx.sync()
    assert int(model.read_tensor("pos", np.int32)[0]) == cap
    for call in (lambda: model.decode(1, 0.25, use_graph=False),
                 lambda: model.decode(1, 0.25, use_graph=True),
                 lambda: model.step_device(0.25),
                 lambda: model.set_position(cap + 1),
                 lambda: model.generate(np.zeros(cap, np.int32), 1, 0.25, use_graph=False)):
        with pytest.raises(iam.IamError) as e:
            call()
        assert e.value.code == -1, e.value
    assert int(model.read_tensor("pos", np.int32)[0]) == cap
    model.set_position(cap)
    with pytest.raises(iam.IamError):
        model.step_device(0.25)
    model.set_position(cap - 1)
    model.decode(1, 0.25, use_graph=False)
    with pytest.raises(iam.IamError):
        model.decode(1, 0.25, use_graph=False)


WIDE = dict(n_layers=1, dim=8192, ffn_dim=4096, n_heads=64, n_kv_heads=8, head_dim=128, vocab=256,
            max_ctx=16, rope_theta=10000.0, norm_eps=1e-5)


def test_wide_model_logits_and_tokens_match_oracle(O, iam, ctx):
    """dim 8192 (64 query heads per 8 KV heads): the norms run as their own
    kernel ahead of the walks and the cutoff reads the first 4096 inputs.
    Logits within 1 ulp of the oracle's at every step (both running free) and
    identical greedy tokens, at effort 0.25 and 1.0."""
    m = iam.Model(ctx, iam.ModelConfig(**WIDE))
    try:
        m.synthesize(3)
        dlog = ctx.empty(WIDE["vocab"], np.float32)
        for effort in (0.25, 1.0):
            orc = O.OracleModel(WIDE, m.read_tensor)
            m.reset_caches()
            toks = O.gen_tokens(3, 91, 6, WIDE["vocab"]).tolist()
            for pos, tok in enumerate(toks):
                m.forward(tok, pos, effort, dlog)
                lg = dlog.read()
                lo = orc.forward(tok, pos, effort)
                assert ulps(lg, lo).max() <= 1, (effort, pos)
                assert int(np.argmax(lg)) == O.argmax(lo), (effort, pos)
        dlog.free()
    finally:
        m.close()


FFN_WIDE = dict(n_layers=1, dim=4096, ffn_dim=14336, n_heads=32, n_kv_heads=8, head_dim=128, vocab=32000,
                max_ctx=64, rope_theta=10000.0, norm_eps=1e-5)


def test_mistral_width_layer_matches_oracle_every_position(O, iam, ctx):
    """One layer at the Mistral-7B widths (FFN 14336, vocabulary 32000): the
    walk grids of these launches carry blocks past the smaller matrices'
    counts, which must still clear their share of the previous launches'
    accumulators.  Logits within 1 ulp of the oracle model's at 12
    consecutive positions (eager steps on the same tokens)."""
    m = iam.Model(ctx, iam.ModelConfig(**FFN_WIDE))
    try:
        m.synthesize(0)
        orc = O.OracleModel(FFN_WIDE, m.read_tensor)
        m.reset_caches()
        dlog = ctx.empty(FFN_WIDE["vocab"], np.float32)
        for pos, tok in enumerate(O.gen_tokens(0, 90, 12, FFN_WIDE["vocab"]).tolist()):
            m.forward(tok, pos, 0.25, dlog)
            assert ulps(dlog.read(), orc.forward(tok, pos, 0.25)).max() <= 1, pos
        dlog.free()
    finally:
        m.close()
