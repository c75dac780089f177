"""GPU parity of the Llama decoder driver (the chatbot.tl composition) against the CPU oracle:
logits within the f32 tolerance, identical greedy tokens, and sampled tokens equal to the
oracle's at the same uniform draws wherever rounding cannot move the choice."""
import json
import os

import numpy as np
import pytest

import oracle
from tl_amd import BackendError
from tl_amd.llama import HipLlama, LlamaConfig, greedy_generate, sampled_generate, synthetic_prompt, synthetic_weights

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
SMALL = LlamaConfig(2, 256, 4, 2, 512, 1000, max_seq=128)


def max_rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.fixture(scope="module")
def small():
    tensors = list(synthetic_weights(SMALL, 11))
    gpu = HipLlama(SMALL)
    gpu.load(tensors)
    cpu = oracle.Llama(SMALL)
    cpu.load(tensors)
    yield gpu, cpu
    gpu.close()
    cpu.close()


def test_prefill_and_decode_logits(small):
    gpu, cpu = small
    prompt = synthetic_prompt(SMALL, 11, 20)
    gpu.configure(kv_f16=False)
    cpu.reset()
    for chunk in (prompt, [5], [999], [0]):
        lg = gpu.forward(chunk)
        lc = cpu.forward(chunk)
        err = max_rel(lg, lc)
        assert err <= 1e-4, f"f32 path logits max-rel-err {err:.2e} after {len(chunk)} tokens"
    assert gpu.position == 23


@pytest.mark.parametrize("use_graph", [True, False])
@pytest.mark.parametrize("penalty", [1.0, 1.1])
def test_greedy_tokens_f32(small, use_graph, penalty):
    gpu, cpu = small
    gpu.configure(kv_f16=False)
    prompt = synthetic_prompt(SMALL, 12, 17)
    got = greedy_generate(gpu, prompt, 24, penalty=penalty, use_graph=use_graph)
    want = cpu.greedy(prompt, 24, penalty=penalty)
    assert list(got) == list(want)


def test_f16_kv_and_f16_prefill_logits(small):
    gpu, cpu = small
    gpu.configure(kv_f16=True)
    prompt = synthetic_prompt(SMALL, 13, 64)
    cpu.reset()
    err = max_rel(gpu.forward(prompt, prefill_f16=True), cpu.forward(prompt))
    assert err <= 1e-2, f"f16 path logits max-rel-err {err:.2e}"
    err = max_rel(gpu.forward([3]), cpu.forward([3]))
    assert err <= 1e-2, f"f16-KV decode logits max-rel-err {err:.2e}"
    gpu.configure(kv_f16=False)


def test_f16_prefill_mfma_attention_chunks():
    """The f16 prefill's MFMA attention in the decoder (head size 64, 8 query heads per KV
    head, as TinyLlama): a 150-token prompt within the f16 tolerance 1e-2 of the oracle, then
    the same prompt in chunks whose lengths are off the kernel's 16-query block, the later
    ones starting at cache positions > 0 -- with per-token RoPE positions the chunked logits
    equal the whole-prompt ones up to f16 rounding of the shorter GEMMs."""
    cfg = LlamaConfig(2, 512, 8, 1, 512, 1000, max_seq=256)
    tensors = list(synthetic_weights(cfg, 41))
    gpu = HipLlama(cfg, kv_f16=True)
    gpu.load(tensors)
    cpu = oracle.Llama(cfg)
    cpu.load(tensors)
    try:
        prompt = synthetic_prompt(cfg, 41, 150)
        cpu.reset()
        err = max_rel(gpu.forward(prompt, prefill_f16=True), cpu.forward(prompt))
        assert err <= 1e-2, f"f16 prefill logits max-rel-err {err:.2e}"
        err = max_rel(gpu.forward([9]), cpu.forward([9]))
        assert err <= 1e-2, f"decode after f16 prefill: logits max-rel-err {err:.2e}"
        gpu.configure(kv_f16=True, rope_per_token=True)
        gpu.reset()
        whole = gpu.forward(prompt, prefill_f16=True)
        gpu.reset()
        for chunk in (prompt[:37], prompt[37:58], prompt[58:]):
            part = gpu.forward(chunk, prefill_f16=True)
        assert gpu.position == 150
        err = max_rel(part, whole)
        assert err <= 1e-3, f"chunked vs whole prompt logits max-rel-err {err:.2e}"
    finally:
        gpu.close()
        cpu.close()


@pytest.mark.parametrize("n", [21, 32, 64])
def test_f16_prefill_one_launch_split_sums(n):
    """Short prompts (32- and 64-row GEMM tiles with K split): the tiles' last-arriving splits
    add the partial slices in-kernel (with the residual for o-proj / down), and the form with
    separate sums -- a split-K sum launch after qkv, the slices added by the next RMSNorm --
    gives bitwise the same logits; both within the f16 tolerance of the oracle."""
    cfg = LlamaConfig(2, 512, 8, 1, 512, 1000, max_seq=256)
    tensors = list(synthetic_weights(cfg, 47))
    gpu = HipLlama(cfg, kv_f16=True)
    gpu.load(tensors)
    cpu = oracle.Llama(cfg)
    cpu.load(tensors)
    lib = gpu.lib
    prev = lib.tl_hip_debug_one_launch_merge(1)
    try:
        prompt = synthetic_prompt(cfg, 47, n)
        cpu.reset()
        ref = cpu.forward(prompt)
        gpu.reset()
        one = gpu.forward(prompt, prefill_f16=True)
        lib.tl_hip_debug_one_launch_merge(0)
        gpu.reset()
        two = gpu.forward(prompt, prefill_f16=True)
        for got in (one, two):
            err = max_rel(got, ref)
            assert err <= 1e-2, f"f16 prefill logits max-rel-err {err:.2e}"
        # the same additions in the same order: bitwise equal logits
        assert np.array_equal(one.view(np.uint32), two.view(np.uint32)), f"max-rel-err {max_rel(one, two):.2e}"
    finally:
        lib.tl_hip_debug_one_launch_merge(prev)
        gpu.close()
        cpu.close()


@pytest.mark.parametrize("kv_f16", [True, False])
def test_long_cache_decode_paths(kv_f16):
    """Caches longer than 4096 positions: decode attention takes the grouped-query split form
    (f16 cache) or the general split form (f32 cache) instead of the one-launch per-head
    kernel; logits against the oracle (1e-2 with the f16 cache, 1e-4 with f32), graph and
    eager greedy tokens equal to the oracle's."""
    cfg = LlamaConfig(2, 512, 8, 1, 512, 1000, max_seq=5000)
    tensors = list(synthetic_weights(cfg, 47))
    gpu = HipLlama(cfg, kv_f16=kv_f16)
    gpu.load(tensors)
    cpu = oracle.Llama(cfg)
    cpu.load(tensors)
    tol = 1e-2 if kv_f16 else 1e-4
    try:
        prompt = synthetic_prompt(cfg, 47, 40)
        cpu.reset()
        err = max_rel(gpu.forward(prompt), cpu.forward(prompt))
        assert err <= tol, f"prefill logits max-rel-err {err:.2e}"
        for t in ([11], [512], [7]):
            err = max_rel(gpu.forward(t), cpu.forward(t))
            assert err <= tol, f"decode logits max-rel-err {err:.2e}"
        if not kv_f16:
            for use_graph in (True, False):
                assert list(greedy_generate(gpu, prompt, 12, use_graph=use_graph)) == list(cpu.greedy(prompt, 12))
    finally:
        gpu.close()
        cpu.close()


@pytest.mark.parametrize("use_graph", [True, False])
def test_decode_attention_share_boundaries(use_graph):
    """The decode step splits each head's cache positions into shares of whole 64-position
    rounds (some empty while the cache is short) whose records the o-projection merges.  200
    greedy tokens after a 59-token prompt cover cache lengths 60-259 -- shares filling,
    starting and empty at 64, 128, 192 and 256 -- and must equal the oracle's (f32 cache)."""
    cfg = LlamaConfig(2, 256, 4, 2, 512, 1000, max_seq=320)
    tensors = list(synthetic_weights(cfg, 53))
    gpu = HipLlama(cfg, kv_f16=False)
    gpu.load(tensors)
    cpu = oracle.Llama(cfg)
    cpu.load(tensors)
    try:
        prompt = synthetic_prompt(cfg, 53, 59)
        got = greedy_generate(gpu, prompt, 200, use_graph=use_graph)
        assert list(got) == list(cpu.greedy(prompt, 200))
    finally:
        gpu.close()
        cpu.close()


@pytest.mark.parametrize("penalty", [1.0, 1.1])
def test_greedy_ties_take_the_last_index(penalty):
    """Every LM-head row equal: all logits tie, and the greedy choice must follow tensor.rs's
    fold (the last maximum) through the per-workgroup candidates and their merge -- the last
    vocabulary index without a penalty; with a penalty each chosen token drops below the
    others and the choice walks down the ties.  Graph and eager tokens equal the oracle's."""
    cfg = LlamaConfig(2, 256, 4, 2, 512, 1000, max_seq=128)
    tensors = []
    for kind, layer, which, payload in synthetic_weights(cfg, 61):
        if kind == "linear" and layer == -1:
            rows = np.ascontiguousarray(payload).reshape(cfg.vocab, -1)
            payload = np.repeat(rows[:1], cfg.vocab, axis=0).reshape(np.shape(payload))
        tensors.append((kind, layer, which, payload))
    gpu = HipLlama(cfg)
    gpu.load(tensors)
    cpu = oracle.Llama(cfg)
    cpu.load(tensors)
    try:
        prompt = synthetic_prompt(cfg, 61, 10)
        want = list(cpu.greedy(prompt, 12, penalty=penalty))
        if penalty == 1.0:
            assert want == [cfg.vocab - 1] * 12
        for use_graph in (True, False):
            assert list(greedy_generate(gpu, prompt, 12, penalty=penalty, use_graph=use_graph)) == want
    finally:
        gpu.close()
        cpu.close()


def test_graph_follows_the_penalty_value(small):
    """The penalty reaches the captured step as a kernel argument: a generate with another
    penalty value must capture again (graph tokens = eager = oracle for 1.1, then 0.5 -- a
    penalty below 1 raises the positive logits of seen tokens, so the ids differ), and a
    longer generate with unchanged settings must replay without a new capture."""
    gpu, cpu = small
    gpu.configure(kv_f16=False)
    prompt = synthetic_prompt(SMALL, 15, 13)
    wants = {}
    for pen in (1.1, 0.5):
        wants[pen] = list(cpu.greedy(prompt, 24, penalty=pen))
    assert wants[1.1] != wants[0.5], "penalties chosen too close to tell the graphs apart"
    builds = lambda: int(gpu.lib.tl_hip_llama_graph_builds(gpu.h))
    for pen in (1.1, 0.5, 1.1):
        b0 = builds()
        # 23 decode steps after the prefill's token: two launches of the 8-step graph and seven
        # of the 1-step graph, both captured for the new penalty
        assert list(greedy_generate(gpu, prompt, 24, penalty=pen, use_graph=True)) == wants[pen]
        assert builds() == b0 + 2
        assert list(greedy_generate(gpu, prompt, 24, penalty=pen, use_graph=False)) == wants[pen]
    b0 = builds()
    for n in (8, 30):   # same settings, fewer and more steps: replays only
        assert list(greedy_generate(gpu, prompt, n, penalty=1.1, use_graph=True)) == \
            list(cpu.greedy(prompt, n, penalty=1.1))
    assert builds() == b0


def _oracle_sampled(cpu, prompt, n, temp, top_p, penalty, draws):
    """chatbot.tl:174-222 on the oracle: penalty, then sample_impl at the given draws.  Yields
    (token, logits) per step."""
    cpu.reset()
    toks, cur = [int(t) for t in prompt], [int(t) for t in prompt]
    for i in range(n):
        logits = cpu.forward(cur)
        if penalty != 1.0:
            logits = oracle.repetition_penalty(logits[None, :], np.array(toks, np.float32), penalty)[0]
        nxt = oracle.sample(logits, temp, top_p, draws[i])
        yield nxt, logits
        toks.append(nxt)
        cur = [nxt]


@pytest.mark.parametrize("use_graph", [True, False])
@pytest.mark.parametrize("temp,top_p,penalty", [(0.7, 0.9, 1.1), (0.1, 0.9, 1.1), (1.5, 0.95, 1.0)])
def test_sampled_tokens_f32(small, use_graph, temp, top_p, penalty):
    """The chatbot's decode as it runs (chatbot.tl:188-189: repetition_penalty(1.1), then
    sample(0.1, 0.9) every token, the first from the prompt's logits) with seeded draws: the
    device's tokens against the oracle's sample_impl at the same draws, step by step.  A step
    may differ only where rounding could move the choice -- top_p or r within 4e-6 plus four
    times the f32 drift of a running sum (sampling_f64.decided) -- and the comparison stops
    there."""
    from sampling_f64 import decided, sample_f64, splitmix64_uniforms
    gpu, cpu = small
    gpu.configure(kv_f16=False)
    prompt = synthetic_prompt(SMALL, 13, 17)
    n, seed = 24, 77
    got = sampled_generate(gpu, prompt, n, temp, top_p, penalty=penalty, seed=seed, use_graph=use_graph)
    draws = splitmix64_uniforms(seed, n)
    for i, (want, logits) in enumerate(_oracle_sampled(cpu, prompt, n, temp, top_p, penalty, draws)):
        if got[i] != want:
            _, margin, drift = sample_f64(logits, temp, top_p, draws[i])
            assert not decided(margin, drift), (i, int(got[i]), want, margin, drift)
            break
    # the same seed replays the same tokens, graph or eager
    again = sampled_generate(gpu, prompt, n, temp, top_p, penalty=penalty, seed=seed, use_graph=not use_graph)
    assert list(again) == list(got)
    if temp >= 0.7:
        other = sampled_generate(gpu, prompt, n, temp, top_p, penalty=penalty, seed=seed + 1, use_graph=use_graph)
        assert list(other) != list(got), "another seed drew the same 24 tokens"


@pytest.mark.parametrize("temp,top_p", [(0.7, 0.9), (1.5, 0.95)])
def test_sampled_tokens_large_vocab(temp, top_p):
    """A vocabulary past 32768 logits: the decode step's sampling keeps its keys in the
    model's global scratch instead of LDS.  Tokens against the oracle at the same draws, graph
    and eager (the same rule on a mismatch as test_sampled_tokens_f32; over 33000 flat
    probabilities the running sums lie ~3e-5 apart, so such steps occur)."""
    from sampling_f64 import decided, sample_f64, splitmix64_uniforms
    cfg = LlamaConfig(1, 128, 2, 1, 256, 33000, max_seq=64)
    tensors = list(synthetic_weights(cfg, 21))
    gpu, cpu = HipLlama(cfg), oracle.Llama(cfg)
    try:
        gpu.load(tensors)
        cpu.load(tensors)
        prompt = synthetic_prompt(cfg, 21, 9)
        n, seed = 12, 31
        draws = splitmix64_uniforms(seed, n)
        runs = [sampled_generate(gpu, prompt, n, temp, top_p, penalty=1.1, seed=seed, use_graph=g) for g in (True, False)]
        assert list(runs[0]) == list(runs[1])
        for i, (want, logits) in enumerate(_oracle_sampled(cpu, prompt, n, temp, top_p, 1.1, draws)):
            if runs[0][i] != want:
                _, margin, drift = sample_f64(logits, temp, top_p, draws[i])
                assert not decided(margin, drift), (i, int(runs[0][i]), want, margin, drift)
                break
    finally:
        gpu.close()
        cpu.close()


def test_sampling_settings_reach_the_graph(small):
    """temp and top_p reach the captured step as kernel arguments: changing either captures
    again, the same settings replay, and greedy decoding after sampling is unchanged."""
    gpu, cpu = small
    gpu.configure(kv_f16=False)
    prompt = synthetic_prompt(SMALL, 14, 9)
    builds = lambda: int(gpu.lib.tl_hip_llama_graph_builds(gpu.h))
    greedy = list(cpu.greedy(prompt, 12, penalty=1.1))
    for temp, top_p, new in ((0.8, 0.9, True), (0.8, 0.9, False), (0.8, 0.5, True), (1.2, 0.5, True)):
        b0 = builds()
        got = sampled_generate(gpu, prompt, 12, temp, top_p, penalty=1.1, seed=5, use_graph=True)
        assert builds() == b0 + (2 if new else 0)
        assert list(got) == list(sampled_generate(gpu, prompt, 12, temp, top_p, penalty=1.1, seed=5,
                                                  use_graph=False))
    assert list(greedy_generate(gpu, prompt, 12, penalty=1.1, use_graph=True)) == greedy
    with pytest.raises(BackendError):
        gpu.set_sampling(float("nan"), 0.9)


@pytest.mark.parametrize("warm,timed", [(5, 20), (8, 3), (1, 9), (16, 7)])
def test_no_capture_after_the_first_graph_call(small, warm, timed):
    """bench.py's decode legs: a warm-up generate of `warm` steps, then a timed generate of
    `timed` steps must only replay, whatever the two lengths are (both graph shapes are
    captured by the first graph-mode call of a key); also for a changed penalty and KV type.
    The tokens of the two calls continue the oracle's greedy sequence."""
    gpu, cpu = small
    prompt = synthetic_prompt(SMALL, 16, 11)
    builds = lambda: int(gpu.lib.tl_hip_llama_graph_builds(gpu.h))
    for kv_f16, pen in ((False, 1.0), (False, 1.1), (True, 1.0)):
        gpu.configure(kv_f16=kv_f16)
        gpu.reset()
        gpu.forward(prompt, want_logits=False)
        first = gpu.sample_greedy(pen, prompt)
        hist = np.concatenate([prompt, [first]]).astype(np.int32)
        b0 = builds()
        w = gpu.generate(first, warm, pen, hist, use_graph=True)
        assert builds() == b0 + 2, "the first graph-mode call captures both graph shapes"
        hist = np.concatenate([hist, w[:-1]]).astype(np.int32)
        t = gpu.generate(int(w[-1]), timed, pen, hist, use_graph=True)
        assert builds() == b0 + 2, f"warm-up {warm} then {timed} steps captured inside the second call"
        if not kv_f16:
            want = list(cpu.greedy(prompt, 1 + warm + timed, penalty=pen))
            assert [first] + list(w) + list(t) == want


def test_failed_activation_grow_leaves_the_model_usable():
    """An allocation failure while the activation buffers grow for a longer call returns
    AllocationError and leaves no stale buffer or captured step behind: the next short call
    allocates again, and greedy tokens (graph and eager) still equal the oracle's."""
    from tl_amd import BackendError
    tensors = list(synthetic_weights(SMALL, 17))
    gpu = HipLlama(SMALL)
    gpu.load(tensors)
    cpu = oracle.Llama(SMALL)
    cpu.load(tensors)
    try:
        prompt = synthetic_prompt(SMALL, 17, 9)
        want = list(cpu.greedy(prompt, 10))
        assert list(greedy_generate(gpu, prompt, 10)) == want        # step captured at 9 tokens
        for fail_after in (0, 3):
            gpu.reset()
            gpu.lib.tl_hip_debug_fail_alloc(fail_after)
            try:
                with pytest.raises(BackendError) as e:
                    gpu.forward(synthetic_prompt(SMALL, 18, 100 + fail_after))
            finally:
                gpu.lib.tl_hip_debug_fail_alloc(-1)
            assert e.value.variant == "AllocationError"
            assert gpu.position == 0
            for use_graph in (True, False):
                assert list(greedy_generate(gpu, prompt, 10, use_graph=use_graph)) == want
    finally:
        gpu.close()
        cpu.close()


def test_position_aware_rope_changes_prefill(small):
    gpu, _ = small
    prompt = synthetic_prompt(SMALL, 14, 12)
    gpu.configure(kv_f16=False, rope_per_token=False)
    a = gpu.forward(prompt)
    gpu.configure(kv_f16=False, rope_per_token=True)
    b = gpu.forward(prompt)
    gpu.configure(kv_f16=False, rope_per_token=False)
    assert not np.allclose(a, b)  # tl_cpu rotates every prompt token by row 0; per-token differs


def test_errors(small):
    gpu, _ = small
    from tl_amd import BackendError
    gpu.reset()
    with pytest.raises(BackendError) as e:
        gpu.forward([SMALL.vocab])
    assert e.value.variant == "IndexOutOfBounds"
    with pytest.raises(BackendError) as e:
        gpu.forward(np.zeros(SMALL.max_seq + 1, np.int32))
    assert e.value.variant == "ArgumentError"


def test_tinyllama_greedy_golden():
    """Full TinyLlama shape: 512-token prompt, 32 greedy tokens equal to the oracle's
    (tests/golden/tinyllama_greedy.json), f32 KV cache, f32 prefill GEMM."""
    with open(os.path.join(HERE, "golden", "tinyllama_greedy.json")) as f:
        gold = json.load(f)
    cfg = LlamaConfig.tinyllama(max_seq=2048)
    prompt = synthetic_prompt(cfg, gold["seed"], gold["prompt_tokens"])
    assert [int(t) for t in prompt[:8]] == gold["prompt_head"]
    m = HipLlama(cfg, kv_f16=False)
    m.load(synthetic_weights(cfg, gold["seed"]))
    got = greedy_generate(m, prompt, len(gold["tokens"]), prefill_f16=False)
    assert list(got) == gold["tokens"]
    # the performance configuration (f16 KV cache, f16-MFMA prefill) on the same model
    m.configure(kv_f16=True)
    got16 = greedy_generate(m, prompt, len(gold["tokens"]), prefill_f16=True)
    # its top-2 logit margins, teacher-forced along the golden tokens (eager forward calls of
    # the same precision class), beside the oracle's: a flip whose margin on either side is
    # within f16 rounding of the logits is a precision event, not a wiring fault
    m.reset()
    lg = m.forward(prompt, prefill_f16=True)
    rows = []
    for i, t in enumerate(gold["tokens"]):
        a, b = (int(v) for v in np.argsort(lg, kind="stable")[::-1][:2])
        rows.append((i, a, b, float(lg[a] - lg[b]), float(lg[a] - lg[t]), gold["top2_margins"][i]))
        lg = m.forward([t], prefill_f16=True)
    m.close()
    print("step  f16 top-1  top-2  f16 margin  f16 top-1 - golden  oracle margin")
    for r in rows:
        print(f"{r[0]:4d} {r[1]:9d} {r[2]:6d} {r[3]:11.3e} {r[4]:19.3e} {r[5]:14.3e}")
    print(f"smallest f16 margin {min(r[3] for r in rows):.3e}, smallest oracle margin "
          f"{min(r[5] for r in rows):.3e}")
    agree = int(np.argmax(np.array(list(got16) + [-1]) != np.array(gold["tokens"] + [-2])))
    print(f"f16 KV / f16 prefill: first {agree} of {len(gold['tokens'])} tokens agree")
    if agree < len(gold["tokens"]):
        i = agree
        r = rows[i]
        pytest.fail(f"f16 path: step {i} chose {int(got16[i])}, the oracle {gold['tokens'][i]}; teacher-forced f16 "
                    f"logits there: top-1 {r[1]}, top-2 {r[2]}, margin {r[3]:.3e}, top-1 minus the golden token "
                    f"{r[4]:.3e}; the oracle's top-2 margin {r[5]:.3e} (an f16 rounding flip has both margins "
                    f"near the f16 logit error, ~1e-3)")


_ROPE_EPI_SMALL = LlamaConfig(2, 512, 8, 1, 512, 1000, max_seq=256)
_ROPE_EPI_WIDE = LlamaConfig(1, 2048, 32, 4, 5632, 1000, max_seq=640)


def _three_qkv_plan(cfg, layer, which):
    # q | k | v in three weights (Q6_K, Q4_K, Q6_K), gate and up alike: a fused prefill layer
    return {"attn_q": 14, "attn_k": 12, "attn_v": 14}.get(which, 12)


@pytest.mark.parametrize("case", ["21-f16", "21-f32-per-token", "77-f16-per-token", "77-f32", "512-wide-f16",
                                  "21-f16-q6qk", "77-f32-q6qk", "21-f16-three", "77-f16-per-token-three"])
def test_f16_prefill_rope_epilogue_matches_rope_kernel(case):
    """The f16 prefill's RoPE and KV append in the [q | k | v] GEMM's epilogue against the
    separate RoPE / KV kernel after a plain GEMM: bitwise the same prefill logits and the same
    logits of a decode step after it (which reads every cache row the prefill wrote), then the
    same for a second 13-token chunk appended at a later cache position.  21
    tokens: 32-row tiles whose last-arriving K split adds the slices and applies RoPE; 77:
    128-row tiles with K split, the sum launch applying it; 512 at TinyLlama's width: 320
    unsplit tiles, the GEMM itself applying it.  f16 and f32 caches, both RoPE position rules;
    Q4_0 weights, and K-quant q | k | v projections stored as two weights (Q6_K q | k, Q4_K v)
    or three, each GEMM rotating and appending its own heads."""
    n, kv = int(case.split("-")[0]), "f16" in case
    cfg = _ROPE_EPI_WIDE if "wide" in case else _ROPE_EPI_SMALL
    gt = _q6_qk_plan if case.endswith("q6qk") else _three_qkv_plan if case.endswith("three") else 2
    tensors = list(synthetic_weights(cfg, 53, ggml_type=gt))
    gpu = HipLlama(cfg, kv_f16=kv)
    gpu.load(tensors, ggml_type=gt)
    lib = gpu.lib
    prev = lib.tl_hip_debug_prefill_rope_epilogue(1)
    try:
        gpu.configure(kv_f16=kv, rope_per_token="per-token" in case)
        prompt = synthetic_prompt(cfg, 53, n)
        got = {}
        for on in (1, 0):
            lib.tl_hip_debug_prefill_rope_epilogue(on)
            assert lib.tl_hip_debug_prefill_rope_epilogue(-1) == on  # the query changes nothing
            assert lib.tl_hip_debug_prefill_rope_epilogue(-1) == on
            gpu.reset()
            pre = gpu.forward(prompt, prefill_f16=True)
            dec = gpu.forward([7])
            # a second prompt chunk at cache positions n + 1 .., then a decode step
            more = gpu.forward(synthetic_prompt(cfg, 54, 13), prefill_f16=True)
            dec2 = gpu.forward([9])
            got[on] = (pre, dec, more, dec2)
        for i, what in enumerate(("prefill", "decode after the prefill", "second chunk at a later position",
                                  "decode after it")):
            a, b = got[1][i], got[0][i]
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{what}: max-rel {max_rel(a, b):.2e}"
        if case == "21-f16":  # and within the f16 tolerance of the oracle (its RoPE position rule)
            cpu = oracle.Llama(cfg)
            cpu.load(tensors)
            try:
                cpu.reset()
                err = max_rel(got[1][0], cpu.forward(prompt))
                assert err <= 1e-2, f"f16 prefill logits max-rel-err {err:.2e}"
            finally:
                cpu.close()
    finally:
        lib.tl_hip_debug_prefill_rope_epilogue(prev)
        gpu.close()


def _q8_handoff_plan(cfg, layer, which):
    # each f16 GEMM input written in the operand order of its reader: Q8_0 and Q4_0 alternate
    return {"attn_q": 8, "attn_k": 8, "attn_v": 8, "attn_output": 2, "ffn_gate": 8, "ffn_up": 8,
            "ffn_down": 2}.get(which, 8)


@pytest.mark.parametrize("plan", ["Q8_0", "q8_handoff", "Q4_K_M", "mixed"])
def test_f16_prefill_weight_mixtures(plan):
    """The f16 prefill (activations passed between GEMMs as f16 operand words, residual and
    SwiGLU in the GEMM epilogues) over weight mixtures: all Q8_0, Q8_0 / Q4_0 alternating
    between producer and reader, llama.cpp's Q4_K_M, and gate / up of different types (the
    unfused path).  Head size 64 with 8 query heads per KV head (MFMA attention).  Logits
    within the f16 tolerance of the oracle, then decode steps."""
    cfg = LlamaConfig(2, 512, 8, 1, 512, 1000, max_seq=128)
    gt = {"Q8_0": 8, "q8_handoff": _q8_handoff_plan, "Q4_K_M": "Q4_K_M", "mixed": _mixed_plan}[plan]
    tensors = list(synthetic_weights(cfg, 43, ggml_type=gt))
    gpu = HipLlama(cfg, kv_f16=True)
    gpu.load(tensors, ggml_type=gt)
    cpu = oracle.Llama(cfg)
    cpu.load(tensors, ggml_type=gt)
    try:
        prompt = synthetic_prompt(cfg, 43, 77)
        cpu.reset()
        err = max_rel(gpu.forward(prompt, prefill_f16=True), cpu.forward(prompt))
        assert err <= 1e-2, f"f16 prefill logits max-rel-err {err:.2e}"
        for t in ([4], [998]):
            err = max_rel(gpu.forward(t), cpu.forward(t))
            assert err <= 1e-2, f"decode logits after the f16 prefill: max-rel-err {err:.2e}"
    finally:
        gpu.close()
        cpu.close()


def _q6_qk_plan(cfg, layer, which):
    # q | k in Q6_K and v in Q4_K: a two-type q | k | v projection with the Q6_K rows first
    return {"attn_q": 14, "attn_k": 14, "attn_v": 12}.get(which, 12)


def _mixed_plan(cfg, layer, which):
    # every grouping case of the loader: q | k | v in three runs, gate and up of different types
    return {"attn_q": 14, "attn_k": 12, "attn_v": 14, "ffn_gate": 14, "ffn_up": 12}.get(which, 12)


@pytest.mark.parametrize("plan", ["Q4_K_M", "mixed", "q6_qk"])
def test_kquant_model_logits_and_tokens(plan):
    """K-quant weights through the whole decoder: llama.cpp's Q4_K_M mixture (Q4_K with Q6_K
    attn_v / ffn_down in some layers and the LM head: the decode step's q | k and v rows in
    one two-type launch), a plan with q/k/v and gate/up of different types (three q | k | v
    runs: one launch each), and Q6_K q | k with a Q4_K v (the two-type launch the other way
    round).  f32 logits within 1e-4 and identical greedy tokens, graph and eager."""
    cfg = LlamaConfig(4, 256, 4, 2, 512, 1000, max_seq=128)
    gt = {"Q4_K_M": "Q4_K_M", "mixed": _mixed_plan, "q6_qk": _q6_qk_plan}[plan]
    tensors = list(synthetic_weights(cfg, 31, ggml_type=gt))
    gpu = HipLlama(cfg)
    gpu.load(tensors, ggml_type=gt)
    cpu = oracle.Llama(cfg)
    cpu.load(tensors, ggml_type=gt)
    try:
        prompt = synthetic_prompt(cfg, 31, 19)
        cpu.reset()
        for chunk in (prompt, [7], [998]):
            err = max_rel(gpu.forward(chunk), cpu.forward(chunk))
            assert err <= 1e-4, f"logits max-rel-err {err:.2e} after {len(chunk)} tokens"
        for use_graph in (True, False):
            got = greedy_generate(gpu, prompt, 16, use_graph=use_graph)
            assert list(got) == list(cpu.greedy(prompt, 16))
    finally:
        gpu.close()
        cpu.close()
