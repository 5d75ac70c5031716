"""The exact end-to-end check of a GPT-2 model against the oracle's (shared
by the float- and integer-attention tests): a prompt, then teacher-forced
decode steps (both sides fed the oracle's greedy token), every step's
logits compared bit for bit, every int16 activation code of every linear's
input compared (the code-flip count per layer and matrix), then the
device-driven greedy loop against the oracle's tokens."""
import numpy as np

SLOTS, SLOT = 49, 3072  # llmq_gpt2_debug_codes / orc set_capture layout
IN_OF_SLOT = [768, 768, 768, 3072] * 12 + [768]
NAMES = ["qkv", "proj", "fc", "fcproj"]
EOT = 50256


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32),
                          np.ascontiguousarray(b, np.float32).view(np.uint32))


def check_decode_exact(torch, orc, model, ref, prompt, steps, label):
    """steps generated tokens (steps - 1 decode forwards, gpt2t.mojo:969-980)
    after `prompt`; asserts zero code flips, bit-identical logits at every
    step and equal device greedy tokens."""
    codes_g = torch.zeros(SLOTS * SLOT, dtype=torch.int16, device="cuda")
    codes_o = np.zeros(SLOTS * SLOT, np.int16)
    model.debug_codes(codes_g)
    ref.set_capture(codes_o)
    flips = np.zeros(SLOTS, np.int64)
    counted = np.zeros(SLOTS, np.int64)
    exact = agree = 0
    worst = 0.0
    print(f"{label}: prefill", flush=True)
    lg, lo = model.forward(prompt, 0), ref.forward(prompt, 0)
    seen = [(lg, lo)]
    toks = []
    pos = len(prompt)
    for i in range(steps - 1):
        nxt = orc.argmax(lo)
        toks.append(nxt)
        lg, lo = model.forward([nxt], pos), ref.forward([nxt], pos)
        pos += 1
        torch.cuda.synchronize()
        g = codes_g.cpu().numpy().reshape(SLOTS, SLOT)
        o = codes_o.reshape(SLOTS, SLOT)
        for s in range(SLOTS):
            k = IN_OF_SLOT[s]
            flips[s] += int(np.count_nonzero(g[s, :k] != o[s, :k]))
            counted[s] += k
        seen.append((lg, lo))
    toks.append(orc.argmax(lo))
    for lg, lo in seen:
        exact += int(bits_equal(lg, lo))
        agree += int(int(np.argmax(lg)) == orc.argmax(lo))
        worst = max(worst, float(np.max(np.abs(lg - lo)) / np.max(np.abs(lo))))
    model.debug_codes(None)
    ref.set_capture(None)
    per_layer = [int(flips[4 * l:4 * l + 4].sum()) for l in range(12)] + [int(flips[48])]
    print(f"{label}: {len(seen)} steps, logits bit-identical {exact}, top-1 agree {agree}, "
          f"max rel err {worst:.1e}; int16 code flips {int(flips.sum())} of {int(counted.sum())} "
          f"(per layer {per_layer[:12]}, head {per_layer[12]})", flush=True)
    gen, _, _ = model.generate(prompt, steps)  # argmax on the GPU, graph per token
    want = toks[:next((i for i, t in enumerate(toks) if t == EOT), len(toks))]
    assert int(flips.sum()) == 0, dict(zip([f"{NAMES[s % 4]}{s // 4}" if s < 48 else "head" for s in range(SLOTS)],
                                          flips.tolist()))
    assert exact == len(seen) and agree == len(seen)
    assert gen.tolist() == want
