"""GGUF residency on the device: weights from a file through tl_hip_gguf_get_quantized /
tl_hip_gguf_get and a whole decoder through tl_hip_llama_load_gguf, against the CPU oracle
on the same bytes."""
import numpy as np
import pytest

import oracle
from tl_amd import GGML_Q4_K, HipTensor
from tl_amd.gguf import GgufFile, write_gguf, write_llama_gguf
from tl_amd.llama import HipLlama, LlamaConfig, greedy_generate, synthetic_prompt, synthetic_weights
from tl_amd.quant import quantize_q4_k, random_q4_0_blocks, random_q6_k_blocks

pytestmark = pytest.mark.gpu


def max_rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def test_get_quantized_and_get(dev, tmp_path):
    rng = np.random.default_rng(41)
    q40 = random_q4_0_blocks(rng, 96, 128)
    q6k = random_q6_k_blocks(rng, 8, 512)
    emb = rng.standard_normal((4, 256)).astype(np.float32)
    qemb = quantize_q4_k(emb)
    h16 = rng.standard_normal((3, 5)).astype(np.float16)
    p = tmp_path / "w.gguf"
    write_gguf(p, [("w40", 2, (96, 128), q40), ("w6k", 14, (8, 512), q6k), ("emb", 12, (4, 256), qemb),
                   ("emb1d", 12, (1024,), qemb), ("h", 1, (3, 5), h16.view(np.uint8)),
                   ("f", 0, (6,), np.arange(6, dtype=np.float32).view(np.uint8))])
    g = GgufFile(p)
    lib = dev.lib
    # tl_qtensor_matmul on the residency built from the mapped bytes
    x = rng.standard_normal((3, 128)).astype(np.float32)
    qa = lib.tl_hip_gguf_get_quantized(g.h, b"w40")
    qb = lib.tl_hip_gguf_get_quantized(g.h, b"w40")  # shared residency, one more reference
    assert qa and qa == qb
    xt = dev.tensor_new(x)
    y = HipTensor(lib.tl_hip_qtensor_matmul(xt.handle, qa), lib).to_numpy()
    assert max_rel(y, oracle.qtensor_matmul(x, q40, 2, 96)) <= 1e-4
    lib.tl_hip_qtensor_release(qa)
    lib.tl_hip_qtensor_release(qb)
    x6 = rng.standard_normal((1, 512)).astype(np.float32)
    q6 = lib.tl_hip_gguf_get_quantized(g.h, b"w6k")
    x6t = dev.tensor_new(x6)
    y6 = HipTensor(lib.tl_hip_qtensor_matmul(x6t.handle, q6), lib).to_numpy()
    assert max_rel(y6, oracle.qtensor_matmul(x6, q6k, 14, 8)) <= 1e-4
    lib.tl_hip_qtensor_release(q6)
    # tl_tensor_map_get: dequantized (bit-exact), F16 converted, F32 as stored
    assert np.array_equal(g.get("emb").to_numpy().view(np.uint32),
                          oracle.dequantize(12, qemb, emb.size).reshape(4, 256).view(np.uint32))
    e1 = g.get("emb1d")
    assert e1.shape == (1024,)
    assert np.array_equal(e1.to_numpy().view(np.uint32), oracle.dequantize(12, qemb, emb.size).view(np.uint32))
    assert np.array_equal(g.get("h").to_numpy(), h16.astype(np.float32))
    assert np.array_equal(g.get("f").to_numpy(), np.arange(6, dtype=np.float32))
    assert not lib.tl_hip_gguf_get_quantized(g.h, b"f")  # F32 has no quantized residency
    assert lib.tl_hip_last_status() == 7
    g.close()


@pytest.mark.parametrize("plan,embed_type", [("Q4_K_M", GGML_Q4_K), (2, 0)])
def test_llama_from_gguf(tmp_path, plan, embed_type):
    """A synthetic decoder written as a GGUF file with the chatbot's tensor names, loaded by
    tl_hip_llama_load_gguf: greedy tokens equal to the oracle's on the same tensors."""
    cfg = LlamaConfig(3, 256, 4, 2, 512, 1000, max_seq=96)
    tensors = list(synthetic_weights(cfg, 43, ggml_type=plan))
    p = tmp_path / "model.gguf"
    stored = write_llama_gguf(p, cfg, tensors, plan, embed_type=embed_type)
    if embed_type:
        t, blocks = stored
        table = oracle.dequantize(t, blocks, cfg.vocab * cfg.d_model).reshape(cfg.vocab, cfg.d_model)
        tensors = [("embedding", -1, 0, table) if k == "embedding" else (k, l, w, pl) for k, l, w, pl in tensors]
    g = GgufFile(p)
    assert g.meta("llama.block_count") == 3
    gpu = HipLlama(cfg)
    gpu.load_gguf(g)
    cpu = oracle.Llama(cfg)
    cpu.load(tensors, ggml_type=plan)
    try:
        prompt = synthetic_prompt(cfg, 43, 13)
        cpu.reset()
        err = max_rel(gpu.forward(prompt), cpu.forward(prompt))
        assert err <= 1e-4, f"logits max-rel-err {err:.2e}"
        got = greedy_generate(gpu, prompt, 12)
        assert list(got) == list(cpu.greedy(prompt, 12))
    finally:
        gpu.close()
        cpu.close()
        g.close()


def test_load_gguf_shape_errors(tmp_path):
    cfg = LlamaConfig(1, 256, 4, 2, 512, 1000, max_seq=32)
    p = tmp_path / "bad.gguf"
    write_gguf(p, [("blk.0.attn_q.weight", 2, (128, 256), bytes(128 * 8 * 18))])
    g = GgufFile(p)
    m = HipLlama(cfg)
    from tl_amd import BackendError
    with pytest.raises(BackendError) as e:
        m.load_gguf(g)
    assert e.value.variant == "ShapeMismatch"
    m.close()
    g.close()
