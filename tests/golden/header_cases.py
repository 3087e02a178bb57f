"""Constructed BF16 GGUF files for the base codec's header ("rest") coder: a BPE tokenizer whose merge
rules build tokens 256.. from earlier ones (the tokenizer-aware form applies), the same with one
malformed merge and with a merged token that is not its pair's concatenation (both fall back to the
lzma form), one rule whose halves are not tokens (the Q8_0 codec's split-position form applies, the
pair form does not), and a file without a tokenizer. Deterministic from their seeds; used by the fixture
writer (make_r2_golden.py --header) and by the tests."""
import numpy as np

from seedpack_amd import gguf

NAMES = ["bpe", "bpe_bad_merge", "bpe_bad_token", "plain", "bpe_split"]


def _bpe(g, nmerge):
    """256 byte tokens, nmerge merged tokens, 6 special tokens, and the merge rules"""
    base = [(chr(33 + i) if i < 94 else chr(0x100 + i)).encode() for i in range(256)]
    toks, merges = list(base), []
    for _ in range(nmerge):
        a = int(g.integers(0, len(toks)))
        b = int(g.integers(0, min(len(toks), 256 + len(merges) // 2 + 1)))
        toks.append(toks[a] + toks[b])
        merges.append(toks[a] + b" " + toks[b])
    toks += [f"<|special_{k}|>".encode() for k in range(6)]
    return toks, merges


def case_file(name):
    """(file bytes, R2 layout of its 2-D BF16 tensors)"""
    g = np.random.Generator(np.random.PCG64(0x4EAD + NAMES.index(name)))
    kv = {"general.architecture": "qwen35", "general.name": f"header case {name}", "general.alignment": 32,
          "qwen35.block_count": 2}
    if name != "plain":
        toks, merges = _bpe(g, 3000)
        if name == "bpe_bad_merge":
            merges[1234] = merges[1234] + b" x"
        if name == "bpe_bad_token":
            toks[256 + 777] = toks[256 + 777] + b"!"
        if name == "bpe_split":             # a rule whose halves are not tokens: the split-position form only
            vocab = set(toks)
            k = next(k for k in range(1000, len(merges)) if len(toks[256 + k]) >= 3 and toks[256 + k][1:] not in vocab)
            merges[k] = toks[256 + k][:1] + b" " + toks[256 + k][1:]
        kv["tokenizer.ggml.model"] = "gpt2"
        kv["tokenizer.ggml.tokens"] = toks
        kv["tokenizer.ggml.token_type"] = [1] * len(toks)
        kv["tokenizer.ggml.merges"] = merges
        kv["tokenizer.ggml.eos_token_id"] = len(toks) - 1
    tensors = [("token_embd.weight", (64, 40), gguf.BF16), ("blk.0.attn_norm.weight", (64,), gguf.F32),
               ("blk.0.attn_q.weight", (64, 64), gguf.BF16), ("blk.1.attn_q.weight", (64, 64), gguf.BF16),
               ("output_norm.weight", (64,), gguf.F32)]
    head, where, size = gguf.header_bytes(kv, tensors)
    data = np.zeros(size, np.uint8)
    data[:len(head)] = np.frombuffer(head, np.uint8)
    for (tname, shape, t), (off, nb) in zip(tensors, where):
        if t == gguf.BF16:
            w = (g.normal(0, 0.02, nb // 2).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
            data[off:off + nb] = w.view(np.uint8)
        else:
            data[off:off + nb] = (1.0 + 0.01 * g.standard_normal(nb // 4)).astype(np.float32).view(np.uint8)
    coded = sorted([(off, nb, shape[0]) for (tname, shape, t), (off, nb) in zip(tensors, where)
                    if t == gguf.BF16 and len(shape) == 2])
    layout = {"size": size, "t": [[o, nb, rl, "bf16"] for o, nb, rl in coded]}
    return data.tobytes(), layout
