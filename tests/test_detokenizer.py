"""Incremental detokenization (CPU).  The reference decodes the whole output
per step (engine/llm_engine.py:151-158) and again for stop strings
(llm_engine.py:213-219); the engine here decodes only a window of the newest
tokens.  Pinned against the full decode of the same ids: for a byte-level
BPE tokenizer (multi-byte characters split over tokens, invalid UTF-8,
special tokens) and for a WordPiece tokenizer (continuation pieces, spaces
cleaned up before punctuation) the streamed deltas concatenate to exactly
the full decode, and the stop-string rule stops on the same token as the
reference's full-decode rule (for stop strings without U+FFFD: the reference
also matches that character against the replacement text of a character
still incomplete at the end of the output)."""

from __future__ import annotations

import random

import pytest

tokenizers = pytest.importorskip("tokenizers")
transformers = pytest.importorskip("transformers")

from litevllm.config import EngineConfig, ModelConfig, SamplingParams  # noqa: E402
from litevllm.engine.llm_engine import LLMEngine  # noqa: E402
from litevllm.engine.sequence import SequenceGroup, SequenceStatus  # noqa: E402
from litevllm.tokenizer import IncrementalDetokenizer, TokenizerGroup  # noqa: E402

CORPUS = [
    "The quick brown fox jumps over the lazy dog.",
    "héllo wörld, naïve café: ¿qué tal? Grüße!",
    "中文分词测试，你好世界。日本語のテキスト。",
    "emoji 🙂🚀 mixed with text, numbers 12345 and punctuation ... !?",
    "def f(x):\n    return x * 2  # code\n",
] * 20


def _byte_level():
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=400, special_tokens=["<eos>", "<|sep|>"],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(CORPUS, trainer)
    return transformers.PreTrainedTokenizerFast(tokenizer_object=tok, eos_token="<eos>")


def _word_piece():
    from tokenizers import Tokenizer, decoders, models, normalizers, pre_tokenizers, trainers
    tok = Tokenizer(models.WordPiece(unk_token="[UNK]"))
    tok.normalizer = normalizers.BertNormalizer(lowercase=True)
    tok.pre_tokenizer = pre_tokenizers.BertPreTokenizer()
    tok.decoder = decoders.WordPiece(cleanup=True)
    trainer = trainers.WordPieceTrainer(vocab_size=300, special_tokens=["[UNK]", "[SEP]"])
    tok.train_from_iterator(CORPUS, trainer)
    return transformers.PreTrainedTokenizerFast(tokenizer_object=tok, unk_token="[UNK]",
                                                sep_token="[SEP]", eos_token="[SEP]")


@pytest.fixture(scope="module", params=["byte_level", "word_piece"])
def tok(request):
    return _byte_level() if request.param == "byte_level" else _word_piece()


def _streams(tok):
    rng = random.Random(0)
    vocab = len(tok)
    out = [tok.encode(t) for t in CORPUS[:5]]
    out += [[rng.randrange(vocab) for _ in range(rng.randrange(1, 60))] for _ in range(40)]
    return out


@pytest.mark.parametrize("skip", [True, False])
def test_token_by_token_deltas_concatenate_to_the_full_decode(tok, skip):
    for ids in _streams(tok):
        d = IncrementalDetokenizer(skip_special_tokens=skip)
        deltas = [d.update(tok, ids[:n]) for n in range(1, len(ids) + 1)]
        assert "".join(deltas) == d.text
        full = tok.decode(ids, skip_special_tokens=skip)
        # the last window may still hold an incomplete character
        assert d.text == full or (full.endswith("\ufffd") and full.startswith(d.text)), ids


def test_updates_of_several_tokens_at_once(tok):
    rng = random.Random(1)
    for ids in _streams(tok):
        d = IncrementalDetokenizer(skip_special_tokens=True)
        n = 0
        while n < len(ids):
            n = min(len(ids), n + rng.randrange(1, 5))
            d.update(tok, ids[:n])
        full = tok.decode(ids, skip_special_tokens=True)
        assert d.text == full or (full.endswith("\ufffd") and full.startswith(d.text))


def _engine(tok):
    eng = LLMEngine(EngineConfig(model_config=ModelConfig("x", load_format="dummy")))
    eng.tokenizer = TokenizerGroup.wrap(tok)
    return eng


def test_stop_strings_stop_on_the_same_token_as_a_full_decode(tok):
    """Reference rule (llm_engine.py:213-219): after each token, stop when a
    stop string occurs in decode(output ids, skip_special_tokens=False)."""
    eng = _engine(tok)
    rng = random.Random(2)
    checked = 0
    for ids in _streams(tok):
        full = tok.decode(ids, skip_special_tokens=False)
        if len(full) < 6:
            continue
        a = rng.randrange(0, len(full) - 3)
        stops = [full[a:a + rng.randrange(1, 4)], "\x00never"]
        if "\ufffd" in stops[0]:
            # the reference's decode of an incomplete character ends in
            # U+FFFD; the window rule waits for the character instead
            continue
        params = SamplingParams(max_tokens=10_000, stop=stops, ignore_eos=True)
        want = next((n for n in range(1, len(ids) + 1)
                     if any(s in tok.decode(ids[:n], skip_special_tokens=False) for s in stops)),
                    None)
        seq = SequenceGroup.create("r", [1, 2, 3], params).seqs[0]
        got = None
        for n, t in enumerate(ids, 1):
            seq.data.append_token(t)
            eng._check_stop(seq, params, t)
            if seq.status == SequenceStatus.FINISHED_STOPPED:
                got = n
                break
        assert got == want, (ids, stops)
        checked += 1
    assert checked > 20


def test_streamed_outputs_and_the_final_text(tok):
    """Streaming: each step's delta_text extends the text; the finished
    output's text is the full decode (the reference's output_text)."""
    eng = _engine(tok)
    eng.stream_text = True
    for ids in _streams(tok)[:20]:
        params = SamplingParams(max_tokens=len(ids), ignore_eos=True)
        sg = SequenceGroup.create("r", [1, 2, 3], params)
        seq = sg.seqs[0]
        deltas = []
        for n, t in enumerate(ids, 1):
            seq.data.append_token(t)
            eng._check_stop(seq, params, t)
            out = eng._build_step_output(sg)
            deltas.append(out.delta_text)
            assert out.finished == (n == len(ids))
        final = tok.decode(ids, skip_special_tokens=True)
        assert out.output_text == final
        assert "".join(deltas) == final
