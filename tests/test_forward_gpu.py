"""The muyo_llm CLI's --forward mode (csrc/forward.cpp), end to end: a Qwen2 GGUF carrying the
tokenizer of tests/golden/bpe_vocab.json and a random 2-layer model, run as a subprocess, against the
oracle following the reference's RunFullModel (src/FullModel.cpp:1093-1290) token by token: the
oracle tokenizer encodes, the oracle model steps every fed token, and the oracle sampler draws
after each feed of a turn's last token and of every generated token but the last.

Checked: the prompt ids, the generated ids, and the exact stdout bytes (text streamed with a split
UTF-8 character held back), greedy and sampled, completion and ChatML chat, an interactive
session of three turns, a context that fills during generation, and the refusals.
"""
import json
import pathlib
import subprocess
import sys

import numpy as np
import pytest

import gguf_writer as gw
import tokenizer as otok

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parents[1]
CLI = ROOT / "muyo-llm_amd" / "muyo_llm"
VOCAB = json.loads((ROOT / "tests" / "golden" / "bpe_vocab.json").read_text(encoding="utf-8"))
SHAPE = dict(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=len(VOCAB["tokens"]),
             max_seq=512)
EOS = VOCAB["tokens"].index("<|im_end|>")
BOS = VOCAB["tokens"].index("<|endoftext|>")
SYSTEM = "You are Qwen, created by Alibaba Cloud. You are a helpful assistant."


@pytest.fixture(scope="module")
def model_file(orc, tmp_path_factory):
    model = orc.Model(**SHAPE)
    model.fill_random(4242)
    path = tmp_path_factory.mktemp("forward") / "chat.gguf"
    gw.qwen2_file(path, model, vocab=VOCAB)
    return model, path


@pytest.fixture(scope="module")
def tok():
    return otok.Tokenizer(VOCAB["tokens"], VOCAB["merges"], VOCAB["token_type"], "qwen2")


def run_cli(path, args, stdin=None):
    cmd = [str(CLI), "--forward", str(path), *args]
    print(f"[cli] {' '.join(cmd[2:])}", flush=True)
    p = subprocess.run(cmd, input=stdin, capture_output=True, timeout=120)
    return p.returncode, p.stdout, p.stderr.decode("utf-8", "replace")


def ids_after(stderr: str, label: str) -> list[int]:
    """The ids on the last line holding `label` (after an interactive session it follows the
    "[chat] you> " prompt on the same line)."""
    line = stderr[stderr.rindex(label):].splitlines()[0]
    return [int(x) for x in line.split(":", 1)[1].split()]


class Reference:
    """RunFullModel's feed/sample loop (src/FullModel.cpp:1096-1206) on the oracle model."""

    def __init__(self, model, tok, ctx, sampler=None):
        model.fill_kv_random(0, 0)
        self.model, self.tok, self.ctx, self.sampler = model, tok, ctx, sampler
        self.fed, self.logits, self.generated = [], None, []
        self.stdout, self.pending = bytearray(), b""

    def feed(self, token) -> bool:
        if len(self.fed) >= self.ctx:
            return False
        _, self.logits, _ = self.model.step(int(token), len(self.fed))
        self.fed.append(int(token))
        return True

    def sample(self) -> int:
        if self.sampler is None:
            best = np.flatnonzero(self.logits == self.logits.max())
            return int(best[0])
        return self.sampler.sample(self.logits.copy(), self.fed)

    def text(self, data: bytes, final=False):
        self.pending += data
        done = 0
        while done < len(self.pending):
            lead = self.pending[done]
            n = 2 if lead & 0xE0 == 0xC0 else 3 if lead & 0xF0 == 0xE0 else 4 if lead & 0xF8 == 0xF0 else 1
            if not final and done + n > len(self.pending):
                break
            done += n
        done = min(done, len(self.pending))
        self.stdout += self.pending[:done]
        self.pending = self.pending[done:]

    def turn(self, tokens, budget):
        self.generated = []
        for t in tokens:
            if not self.feed(t):
                return
        for _ in range(budget):
            nxt = self.sample()
            self.generated.append(nxt)
            if not self.tok.is_special(nxt):
                self.text(self.tok.token_bytes(nxt))
            if not self.feed(nxt):
                break
            if nxt == EOS:
                break

    def finish(self) -> bytes:
        self.text(b"", final=True)
        return bytes(self.stdout) + b"\n"


def test_completion_greedy(model_file, tok, orc):
    model, path = model_file
    prompt = "Hello world! It's a test of the tokenizer, isn't it?"
    rc, out, err = run_cli(path, ["-p", prompt, "-n", "24", "--ctx", "512"])
    assert rc == 0, err
    want_prompt = tok.encode(prompt)
    assert ids_after(err, "[forward] prompt tokens") == want_prompt
    ref = Reference(model, tok, 512)
    ref.turn(want_prompt, 24)
    assert ids_after(err, "[forward] generated") == ref.generated
    assert out == ref.finish()


def test_completion_from_ids_and_default_bos(model_file, tok):
    model, path = model_file
    rc, out, err = run_cli(path, ["--tokens", "840,826,0", "-n", "6", "--ctx", "512"])
    assert rc == 0, err
    assert ids_after(err, "[forward] prompt tokens") == [840, 826, 0]
    ref = Reference(model, tok, 512)
    ref.turn([840, 826, 0], 6)
    assert ids_after(err, "[forward] generated") == ref.generated
    rc, out, err = run_cli(path, ["--tokens", ",", "-n", "3", "--ctx", "512"])
    assert rc == 0, err
    assert ids_after(err, "[forward] prompt tokens") == [BOS]


def test_chat_sampled(model_file, tok, orc):
    model, path = model_file
    flags = ["--temp", "0.9", "--top-k", "20", "--top-p", "0.9", "--repeat-penalty", "1.3", "--repeat-last-n", "16",
             "--seed", "7"]
    rc, out, err = run_cli(path, ["--chat", "-p", "Tell me about Paris.", "-n", "20", "--ctx", "512", *flags])
    assert rc == 0, err
    sampler = orc.Sampler(temperature=0.9, top_k=20, top_p=0.9, repeat_penalty=1.3, repeat_last_n=16, seed=7)
    ref = Reference(model, tok, 512, sampler)
    framed = "<|im_start|>system\n" + SYSTEM + "<|im_end|>\n<|im_start|>user\nTell me about Paris.<|im_end|>\n" \
             "<|im_start|>assistant\n"
    ref.turn(tok.encode(framed), 20)
    assert ids_after(err, "[forward] generated") == ref.generated
    assert out == ref.finish()


def test_interactive_turns(model_file, tok, orc):
    """The system turn, then three user lines (an empty one skipped) and /exit: each later turn
    starts with a newline after the assistant's reply, the held-back last token of a turn is fed
    first, and the seeded sampler draws once per generated token."""
    model, path = model_file
    stdin = "Hello\n\nHow are you?\nBye\n/exit\nignored\n".encode()
    flags = ["--temp", "0.7", "--seed", "11", "--system", "Be brief."]
    rc, out, err = run_cli(path, ["-i", "-n", "10", "--ctx", "512", *flags], stdin=stdin)
    assert rc == 0, err
    ref = Reference(model, tok, 512, orc.Sampler(temperature=0.7, seed=11))
    for t in tok.encode("<|im_start|>system\nBe brief.<|im_end|>\n"):
        ref.feed(t)
    for i, line in enumerate(["Hello", "How are you?", "Bye"]):
        ref.stdout += b"\n"
        prefix = "" if i == 0 else "\n"
        ref.turn(tok.encode(prefix + "<|im_start|>user\n" + line + "<|im_end|>\n<|im_start|>assistant\n"), 10)
    assert ids_after(err, "[forward] generated") == ref.generated
    assert out == ref.finish()
    assert err.count("[chat] you>") == 5


def test_context_fills_during_generation(model_file, tok):
    model, path = model_file
    prompt = tok.encode("The quick brown fox jumps over the lazy dog. " * 3)
    ctx = len(prompt) + 10
    rc, out, err = run_cli(path, ["--tokens", ",".join(map(str, prompt)), "-n", "40", "--ctx", str(ctx)])
    assert rc == 0, err
    ref = Reference(model, tok, ctx)
    ref.turn(prompt, 40)
    got = ids_after(err, "[forward] generated")
    assert len(got) == 11 and got == ref.generated


def test_refusals(model_file, tok):
    _, path = model_file
    rc, _, err = run_cli(path, ["--tokens", "1,2,3,4", "--ctx", "4"])
    assert rc == 1 and "prompt is 4 tokens, the cache holds 4" in err
    rc, _, err = run_cli(path, ["--bogus"])
    assert rc == 2 and "unknown --forward option" in err
    rc, _, err = run_cli(path, ["-n"])
    assert rc == 1 and "needs a value" in err
    rc, _, err = run_cli(pathlib.Path("/nonexistent.gguf"), ["-n", "1"])
    assert rc == 1 and "[fail]" in err
