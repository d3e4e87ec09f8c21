"""The reference's own Qwen 3.5 9B configuration at full size
(nm/src/qwen35.hpp:62-88): 32 layers (24 gated delta-net + 8 GQA), d_model
4096, SwiGLU 12288, vocabulary 248320, untied output.weight, 16 query / 4 K/V
attention heads of 256 channels with a quarter of them rotating (RoPE base
1e7), 16 delta-net key heads over 32 value heads. Synthetic Q8_0 weights (the
reference publishes no checkpoint here); the GPU path and the oracle run the
same model bytes: a 48-token prefill and 8 greedy passes, logits bit for bit.
The 256-wide heads take the per-row attention kernels; the rest of the step is
the decode path of the benchmark's model."""
import os
import time

import numpy as np
import pytest

import hero_amd
import oracle
from gpu_util import bits

pytestmark = pytest.mark.gpu

QWEN35_9B = hero_amd.HybridShape(vocab=248320, d_model=4096, layers=32, ffn=12288, q_heads=16, kv_heads=4, head_dim=256,
                                 key_heads=16, value_heads=32, rope_base=1e7)


def say(msg):
    print(msg, flush=True)


@pytest.mark.timeout(900)
def test_qwen35_9b_config_matches_oracle():
    oracle.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    t = time.perf_counter()
    image = hero_amd.synthetic_gguf_image(QWEN35_9B, seed=90000, ctx=1024, tied=False)
    say(f"[9b] synthetic GGUF image {image.nbytes / 1e9:.2f} GB in {time.perf_counter() - t:.1f} s")
    model = hero_amd.Qwen35Model.open_image(image)
    ref = oracle.Model(image=image)
    try:
        d = model.dims
        assert (d.vocab, d.head_dim, d.rotary_dims, d.q_heads, d.kv_heads, d.key_heads, d.value_heads, d.tied) == (248320, 256, 64, 16, 4, 16, 32, 0)
        prompt = np.random.default_rng(90001).integers(0, 248320, 48).astype(np.int32)
        t = time.perf_counter()
        expect = ref.forward_ids(prompt)
        ids = [int(np.argmax(expect))]
        last = expect
        for _ in range(8):
            last = ref.forward_ids([ids[-1]])
            ids.append(int(np.argmax(last)))
        say(f"[9b] oracle: prefill + 8 passes in {time.perf_counter() - t:.1f} s; ids {ids}")
        state = model.new_state(256)
        lg = model.forward(state, ids=prompt)
        assert np.array_equal(bits(lg.values), bits(expect))
        got, glast = model.decode_greedy(state, lg.argmax(), 8, want_logits=True)
        assert [lg.argmax()] + [int(i) for i in got] == ids
        assert np.array_equal(bits(glast.values), bits(last))
        say("[9b] GPU prefill logits, greedy ids and last logits equal the oracle's")
        state.close()
    finally:
        model.close()
        ref.close()
