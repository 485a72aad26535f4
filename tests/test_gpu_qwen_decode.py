"""The full-size decode workloads on the GPU against the reference's own CPU engine.

Qwen2.5-1.5B-shaped decoder (28 layers, hidden 1536, FFN 8960, 12/2 heads,
q/k/v bias, tied 151936-token head, random permutations): a 2048-id prompt,
then 64 greedy tokens. Llama-3-8B-shaped decoder (32 layers, hidden 4096,
FFN 14336, 32/8 heads, untied 128256-token head): a 3968-id prompt, then 128
greedy tokens, so the last one attends over position 4095 of a 4096-position
cache. Random-init zero-mean Q4 weights, seeded.

The reference side is a fixture (tests/golden/full_decode.npz, written by
tests/golden/make_golden.py full from oracle/_ref): the reference reads the
prompt with sml_prefill under SML_PROMPT_SB=0 (equal to stepping, bit for
bit), then decodes with sml_forward; per step it keeps the greedy id, a
digest of the logits' bytes, the top 8 and the logits' spread.

- exact mode: the GPU reads the prompt and greedy-decodes on its own argmax;
  every step's logits have the reference's digest (equal bit for bit), so the
  ids are identical at every step.
- fast mode (the default kernels, the throughput path): teacher-forced on the
  reference's ids, graded as the reference grades its own GPU path
  (sml/sml-gpu-fwd.c:2565-2601) against the exact run's logits: per-step
  logit correlation, and top-1 agreement where a different top-1 counts only
  as a tie within 1% of a logit standard deviation. Its GEMVs reduce over 64
  lanes and its attention over splits, so activations differ from the
  reference's in the last bits; an int8 code that rounds the other way moves
  the next product by one step, and over 28-32 layers such flips add up
  (measured: mean correlation 0.9998 / 0.9989, top-1 agreement 62/64 and
  119/128 with the disagreements 0.011-0.078 s.d. apart). The bar is the
  measured level: worst correlation >= 0.998, top-1 agreement (ties
  included) >= 90%.
"""
import hashlib
import importlib.util
import os

import numpy as np
import pytest

import sheep_amd as sa

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
mg = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mg)
FIX_PATH = os.path.join(HERE, "golden", "full_decode.npz")


def digest(lg):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(lg, np.float32).tobytes()).digest()[:16], np.uint8)


def scratch(tmp_path):
    for d in ("/dev/shm", str(tmp_path)):
        try:
            if os.path.isdir(d) and os.statvfs(d).f_bavail * os.statvfs(d).f_frsize > 8e9:
                return d
        except OSError:
            pass
    return str(tmp_path)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["qwen", "llama"])
def test_full_decode_exact_then_fast(tmp_path, name):
    FIX = np.load(FIX_PATH)
    c = mg.FULL[name]
    V, P, S = c["model"]["n_vocab"], c["prompt"], c["steps"]
    toks = FIX[f"{name}_tokens"]
    assert len(set(toks.tolist())) >= 8, f"the reference's greedy ids are not diverse: {toks}"
    path = os.path.join(scratch(tmp_path), f"sml_full_{name}.ssf")
    try:
        sa.synth_model(path, **c["model"])
        with open(path, "rb") as f:
            h = hashlib.sha256()
            for blk in iter(lambda: f.read(1 << 24), b""):
                h.update(blk)
        assert h.digest() == FIX[f"{name}_sha"].tobytes(), "synthetic model drifted from the fixture's"
        prompt = mg.full_prompt(name)
        n_ctx = P + S

        # exact mode: free-running greedy, every step's logits bit-equal to the reference's
        d = sa.Decoder(path, n_ctx=n_ctx, exact=True)
        exact_logits = []
        try:
            assert d.exact
            lg = d.prefill(prompt, 0, V)
            for i in range(S):
                assert (digest(lg) == FIX[f"{name}_digest"][i]).all(), (
                    f"{name} step {i}: logits differ from the reference's; top ids {np.argsort(-lg)[:4]} "
                    f"vs {FIX[f'{name}_top'][i][:4]}")
                tok = int(np.argmax(lg))
                assert tok == int(toks[i]), f"{name} step {i}: gpu {tok} reference {int(toks[i])}"
                exact_logits.append(lg)
                if i + 1 < S:
                    lg = d.step(tok, P + i, V)
        finally:
            d.close()

        # fast mode: teacher-forced on the reference's ids, graded against the exact logits
        d = sa.Decoder(path, n_ctx=n_ctx)
        corrs, ties, outside = [], 0, []
        try:
            lg = d.prefill(prompt, 0, V)
            for i in range(S):
                ref = exact_logits[i]
                corrs.append(float(np.corrcoef(lg, ref)[0, 1]))
                a, g = int(np.argmax(ref)), int(np.argmax(lg))
                if a != g:
                    gap = (float(ref[a]) - float(ref[g])) / float(ref.std())
                    if gap <= 0.01:
                        ties += 1
                    else:
                        outside.append((i, a, g, round(gap, 4)))
                if i + 1 < S:
                    lg = d.step(int(toks[i]), P + i, V)
        finally:
            d.close()
        print(f"{name} fast mode over {S} steps: mean logit corr {np.mean(corrs):.6f}, worst {min(corrs):.6f}, "
              f"top-1 agree {S - len(outside)}/{S} ({ties} ties), outside the tie rule: {outside}")
        assert min(corrs) >= 0.998, min(corrs)
        assert S - len(outside) >= 0.9 * S, outside
    finally:
        if os.path.exists(path):
            os.unlink(path)
