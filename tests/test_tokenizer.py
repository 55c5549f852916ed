"""The C ABI's tokenizer (oxb_tokenizer_*, host code) against HuggingFace
`tokenizers` built the way the reference builds it (rs/tokenizer.rs:22-90:
models.BPE(vocab, merges, unk_token="<unk>"), ByteLevel pre-tokenizer and
decoder with add_prefix_space False, trim_offsets True, use_regex False).

The reference pins tokenizers 0.21.4 (packages/rust/Cargo.lock); the Python
package here is 0.22.x, whose BPE merge order and byte-level mapping are the
same algorithm.  The vocabulary and merges come from a BPE trained in the test
on a fixed corpus, so the merges are real ranked merges (multi-byte words,
'Ġ'-prefixed pieces, UTF-8 sequences), written into a GGUF that both sides
read: the ids, per-token decodes and chat templates must be identical.
"""
import ctypes as C
import random

import numpy as np
import pytest

from helpers import pkg, synth

tokenizers = pytest.importorskip("tokenizers")
from tokenizers import decoders, models, pre_tokenizers, trainers  # noqa: E402

SPECIALS = ["<|begin_of_text|>", "<|end_of_text|>", "<|start_header_id|>", "<|end_header_id|>",
            "<|eot_id|>"]

CORPUS = [
    "The quick brown fox jumps over the lazy dog.",
    "BitNet b1.58 uses ternary weights {-1, 0, +1} and 8-bit activations.",
    "Ternary matrix-vector products stream two bits per weight from memory.",
    "def forward(self, ids):\n    return self.lm_head(self.norm(x))\n",
    "Les réseaux de neurones ternaires réduisent la mémoire.",
    "Die Gewichte werden beim Laden einmal umgepackt.",
    "日本語のテキストもバイト単位で符号化されます。",
    "Числа: 1234567890, 3.14159, -2.71828.",
    "emoji: 🙂🚀✨ and symbols: ∑ ∫ √ ≈ ≠ ≤ ≥",
    "tabs\tand\nnewlines\r\n  double  spaces   triple",
    "<|start_header_id|>user<|end_header_id|> is how a chat turn begins",
]


def _train(vocab_size=700):
    tok = tokenizers.Tokenizer(models.BPE(unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    tr = trainers.BpeTrainer(vocab_size=vocab_size, min_frequency=1, show_progress=False,
                             initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(CORPUS * 20, trainer=tr)
    vocab = tok.get_vocab()
    tokens = [t for t, _ in sorted(vocab.items(), key=lambda kv: kv[1])]
    merges = [" ".join(m) for m in tok.model.get_merges()] if hasattr(tok.model, "get_merges") \
        else None
    if merges is None:   # older bindings: read the merges from the saved model
        import json
        merges = json.loads(tok.to_str())["model"]["merges"]
        merges = [m if isinstance(m, str) else " ".join(m) for m in merges]
    return tokens, merges


def _reference(tokens, merges):
    """The tokenizer as rs/tokenizer.rs:40-84 builds it."""
    vocab = {t: i for i, t in enumerate(tokens)}   # a repeated token keeps its last id
    pairs = [tuple(m.split(" ", 1)) for m in merges if " " in m]
    tk = tokenizers.Tokenizer(models.BPE(vocab=vocab, merges=pairs, unk_token="<unk>"))
    tk.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, trim_offsets=True,
                                                use_regex=False)
    tk.decoder = decoders.ByteLevel(add_prefix_space=False, trim_offsets=True, use_regex=False)
    return tk


class Native:
    def __init__(self, path):
        self.L = pkg.lib()
        self.t = self.L.oxb_tokenizer_load(path.encode())
        if not self.t:
            raise pkg.NativeError(self.L.oxb_last_error().decode())

    def encode(self, text, bos=False):
        n = self.L.oxb_tokenizer_encode(self.t, text.encode(), int(bos), None, 0)
        assert n >= 0, self.L.oxb_last_error()
        ids = (C.c_int32 * max(n, 1))()
        assert self.L.oxb_tokenizer_encode(self.t, text.encode(), int(bos), ids, n) == n
        return list(ids[:n])

    def decode_one(self, i):
        n = self.L.oxb_tokenizer_decode_one(self.t, i, None, 0)
        buf = C.create_string_buffer(n + 1)
        self.L.oxb_tokenizer_decode_one(self.t, i, buf, n + 1)
        return buf.raw[:n].decode("utf-8")

    def chat(self, msgs):
        roles = (C.c_char_p * len(msgs))(*[r.encode() for r, _ in msgs])
        conts = (C.c_char_p * len(msgs))(*[c.encode() for _, c in msgs])
        n = self.L.oxb_tokenizer_chat(self.t, roles, conts, len(msgs), None, 0)
        assert n >= 0, self.L.oxb_last_error()
        ids = (C.c_int32 * max(n, 1))()
        self.L.oxb_tokenizer_chat(self.t, roles, conts, len(msgs), ids, n)
        return list(ids[:n])

    def info(self):
        out = (C.c_int32 * 5)()
        assert self.L.oxb_tokenizer_info(self.t, out) == 0
        return list(out)

    def close(self):
        self.L.oxb_tokenizer_free(self.t)


@pytest.fixture(scope="module")
def trained(tmp_path_factory):
    tokens, merges = _train()
    tokens = tokens + SPECIALS
    path = str(tmp_path_factory.mktemp("tok") / "bpe.gguf")
    bos = tokens.index("<|begin_of_text|>")
    synth.write_tokenizer_gguf(path, tokens, merges, bos=bos, eos=tokens.index("<|end_of_text|>"))
    nat = Native(path)
    yield tokens, merges, nat, _reference(tokens, merges)
    nat.close()


def _texts(seed=0, n=300):
    rng = random.Random(seed)
    words = " ".join(CORPUS).split() + ["", " ", "  ", "\n", "<|eot_id|>", "ŉ", " ", "é"]
    out = list(CORPUS) + ["", " ", "a", "ab", "  leading", "trailing  ", "<|eot_id|>",
                          "<|start_header_id|>assistant<|end_header_id|>\n\n"]
    scripts = [(0x20, 0x7e), (0xa0, 0x17f), (0x400, 0x45f), (0x3040, 0x30ff), (0x4e00, 0x4fff),
               (0x1f300, 0x1f64f)]
    for _ in range(n):
        if rng.random() < 0.5:
            out.append(" ".join(rng.choice(words) for _ in range(rng.randint(1, 12))))
        else:
            lo, hi = rng.choice(scripts)
            out.append("".join(chr(rng.randint(lo, hi)) for _ in range(rng.randint(1, 20))))
    return out


def test_merges_were_trained(trained):
    tokens, merges, _, ref = trained
    assert len(merges) > 300
    # the reference BPE really merges: a corpus sentence is far fewer tokens than bytes
    s = CORPUS[0]
    assert len(ref.encode(s, add_special_tokens=False).ids) < len(s.encode()) / 2


def test_encode_matches_hf_bpe(trained):
    _, _, nat, ref = trained
    for text in _texts():
        want = ref.encode(text, add_special_tokens=False).ids
        assert nat.encode(text) == want, repr(text)


def test_encode_prepends_bos(trained):
    tokens, _, nat, ref = trained
    bos = tokens.index("<|begin_of_text|>")
    assert nat.encode("hello world", bos=True) == [bos] + ref.encode("hello world").ids
    assert nat.encode("", bos=True) == [bos]
    assert nat.info()[:2] == [bos, tokens.index("<|end_of_text|>")]


def test_decode_one_matches_hf_for_every_id(trained):
    tokens, _, nat, ref = trained
    for i in range(len(tokens)):
        assert nat.decode_one(i) == ref.decode([i], skip_special_tokens=True), (i, tokens[i])
    # special tokens are ordinary vocabulary entries: their text comes back
    assert nat.decode_one(tokens.index("<|eot_id|>")) == "<|eot_id|>"
    # a lone UTF-8 lead byte is one U+FFFD; out-of-range ids are empty
    assert nat.decode_one(tokens.index("â")) == "�"
    assert nat.decode_one(len(tokens) + 5) == ""


def test_llama3_chat_template(trained):
    """rs/tokenizer.rs:177-193 over the reference tokenizer's encodes."""
    tokens, _, nat, ref = trained
    sh, eh, eot = (tokens.index(t) for t in ("<|start_header_id|>", "<|end_header_id|>",
                                              "<|eot_id|>"))
    bos = tokens.index("<|begin_of_text|>")
    msgs = [("system", "You are terse."), ("user", "Dis bonjour 🙂"), ("assistant", "bonjour"),
            ("user", "again")]
    enc = lambda s: ref.encode(s, add_special_tokens=False).ids   # noqa: E731
    want = [bos]
    for r, c in msgs:
        want += [sh] + enc(r) + [eh] + enc("\n\n" + c) + [eot]
    want += [sh] + enc("assistant") + [eh] + enc("\n\n")
    assert nat.chat(msgs) == want
    assert nat.info()[2] == eot and nat.info()[3] == -1


def test_chatml_and_plain_templates(tmp_path):
    base = [synth._byte_alphabet()[b] for b in range(256)]
    enc_ref = lambda tk, s: tk.encode(s, add_special_tokens=False).ids   # noqa: E731
    # ChatML (rs/tokenizer.rs:196-215) when <|im_start|> and <|im_end|> exist
    toks = base + ["<s>", "</s>", "<|im_start|>", "<|im_end|>"]
    p = synth.write_tokenizer_gguf(str(tmp_path / "chatml.gguf"), toks, [], bos=256, eos=257)
    nat, ref = Native(p), _reference(toks, [])
    msgs = [("user", "hi"), ("assistant", "yo")]
    want = [256]
    for r, c in msgs:
        want += [258] + enc_ref(ref, f"{r}\n{c}") + [259] + enc_ref(ref, "\n")
    want += [258] + enc_ref(ref, "assistant\n")
    assert nat.chat(msgs) == want
    assert nat.info()[3] == 259
    nat.close()
    # neither template's specials: contents joined by newlines, BOS first (:171-175)
    toks = base + ["<s>", "</s>"]
    p = synth.write_tokenizer_gguf(str(tmp_path / "plain.gguf"), toks, [], bos=256, eos=257)
    nat, ref = Native(p), _reference(toks, [])
    assert nat.chat(msgs) == [256] + enc_ref(ref, "hi\nyo")
    nat.close()


def test_merge_order_is_rank_then_leftmost(tmp_path):
    """Hand-made merges whose result depends on the order: 'b c' (rank 0)
    beats 'a b' (rank 1) on "abc"; equal ranks resolve leftmost first on
    "aaa"; a merge made stale by an earlier one is skipped."""
    base = [synth._byte_alphabet()[b] for b in range(256)]
    toks = base + ["bc", "ab", "aa", "abc", "aabc"]
    merges = ["b c", "a b", "a a", "a bc", "aa bc"]
    p = synth.write_tokenizer_gguf(str(tmp_path / "m.gguf"), toks, merges)
    nat, ref = Native(p), _reference(toks, merges)
    for text in ["abc", "aaa", "aabc", "aaabc", "abcabc", "bcab", "abab", "aaaa", "cab"]:
        assert nat.encode(text) == ref.encode(text, add_special_tokens=False).ids, text
    nat.close()


def test_bad_merges_and_unknown_bytes(tmp_path):
    base = [synth._byte_alphabet()[b] for b in range(256)]
    # a merge whose result is not in the vocabulary fails the build (as HF's)
    p = synth.write_tokenizer_gguf(str(tmp_path / "bad.gguf"), base, ["a b"])
    with pytest.raises(pkg.NativeError, match="out of vocabulary"):
        Native(p)
    with pytest.raises(Exception):
        _reference(base, ["a b"])
    # a byte with no symbol: encode fails without "<unk>", maps to it with one
    no_z = [t for t in base if t != "z"]
    p = synth.write_tokenizer_gguf(str(tmp_path / "noz.gguf"), no_z, [])
    nat = Native(p)
    assert nat.L.oxb_tokenizer_encode(nat.t, b"az", 0, None, 0) == -1
    nat.close()
    with_unk = no_z + ["<unk>"]
    p = synth.write_tokenizer_gguf(str(tmp_path / "unk.gguf"), with_unk, [])
    nat, ref = Native(p), _reference(with_unk, [])
    assert nat.encode("azz") == ref.encode("azz", add_special_tokens=False).ids \
        == [with_unk.index("a"), with_unk.index("<unk>"), with_unk.index("<unk>")]
    nat.close()


def test_repeated_token_keeps_its_last_id(tmp_path):
    base = [synth._byte_alphabet()[b] for b in range(256)]
    toks = base + ["ab", "xy", "ab"]   # "ab" at 256 and 258
    p = synth.write_tokenizer_gguf(str(tmp_path / "dup.gguf"), toks, ["a b"])
    nat, ref = Native(p), _reference(toks, ["a b"])
    assert nat.encode("ab") == ref.encode("ab", add_special_tokens=False).ids == [258]
    assert nat.decode_one(256) == ref.decode([256], skip_special_tokens=True) == ""
    assert nat.decode_one(258) == "ab"
    nat.close()


def test_synthetic_model_vocab_has_no_merges():
    """The synthetic model files carry no merges, so text encodes byte by byte
    (generate("ab") prefills [BOS, 97, 98]); the words of the synthetic
    vocabulary are reachable only as model outputs."""
    path = synth.cached_gguf(synth.small_config(), seed=7)
    nat = Native(path)
    assert nat.encode("ab", bos=True) == [256, 97, 98]
    assert nat.decode_one(300) == " an" and nat.decode_one(260) == "<|eot_id|>"
    nat.close()
