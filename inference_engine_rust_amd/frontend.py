"""Text front end of the token loop: tokenizer, prompt styles and the greedy command line
(src/tokenizer/backend.rs, src/chat_prompt.rs, src/main.rs), over the device session.

The token loop itself (prefill, decode, logits, argmax or temperature sampling) runs through the
C ABI (`engine`); this module only turns text into token ids and back. The tokenizers are the
same third-party libraries the reference binds: SentencePiece for `.model` files (the Rust
`sentencepiece` crate wraps the same C++ library) and Hugging Face `tokenizers` for `.json`.

    python -m inference_engine_rust_amd -m model.gguf -t tokenizer.model -n 32 "Rust will rule the"
"""
from __future__ import annotations

import argparse
import os
import sys
from dataclasses import dataclass
from enum import Enum

from . import engine as E


_ERR_MODEL = 6  # EngineError::Model (IEK_ERR_MODEL)


class TokenizerError(RuntimeError):
    """EngineError::Tokenizer (src/error.rs)."""


@dataclass
class TokenizerPromptConfig:
    """TokenizerPromptConfig (src/model_config.rs:8-60), read from the GGUF by the library."""
    add_bos_token: bool = False
    add_eos_token: bool = False
    bos_token_id: int = 1
    eos_token_id: int = 2

    @classmethod
    def from_model(cls, model: "E.LoadedModel") -> "TokenizerPromptConfig":
        t = model.tokenizer_prompt()
        return cls(bool(t.add_bos_token), bool(t.add_eos_token), int(t.bos_token_id), int(t.eos_token_id))


class Tokenizer:
    """Tokenizer (src/tokenizer/backend.rs:14-141): SentencePiece `.model` or Hugging Face
    `tokenizer.json` (chosen by the `.json` extension, case-insensitive)."""

    def __init__(self, backend: str, inner):
        self._backend = backend
        self._inner = inner
        self._id_to_piece: dict[int, str] = {}  # SentencePiece pieces seen by encode (for decode)

    @classmethod
    def load_from_file(cls, path: str) -> "Tokenizer":
        if os.path.splitext(path)[1].lower() == ".json":
            from tokenizers import Tokenizer as HfTokenizer
            try:
                return cls("hf", HfTokenizer.from_file(path))
            except Exception as e:  # the library raises its own exception types
                raise TokenizerError(f"failed to load Hugging Face tokenizer.json: {e}") from e
        import sentencepiece as spm
        try:
            return cls("spm", spm.SentencePieceProcessor(model_file=path))
        except Exception as e:
            raise TokenizerError(f"failed to load SentencePiece tokenizer: {e}") from e

    def encode(self, text: str) -> list[int]:
        """Token ids of `text`, no special tokens added (backend.rs:64-81)."""
        if self._backend == "hf":
            return list(self._inner.encode(text, add_special_tokens=False).ids)
        ids = self._inner.encode(text, out_type=int)
        for i in ids:
            self._id_to_piece[i] = self._inner.id_to_piece(i)
        return list(ids)

    def encode_with_prompt_config(self, text: str, cfg: TokenizerPromptConfig) -> list[int]:
        """encode + optional BOS in front and EOS at the end (backend.rs:83-96)."""
        ids = self.encode(text)
        if cfg.add_bos_token:
            ids.insert(0, cfg.bos_token_id)
        if cfg.add_eos_token:
            ids.append(cfg.eos_token_id)
        return ids

    def decode_piece_ids(self, ids) -> str:
        """Text of token ids (backend.rs:52-62)."""
        ids = [int(i) for i in ids]
        if self._backend == "hf":
            return self._inner.decode(ids, skip_special_tokens=False)
        return self._inner.decode(ids)

    def decode(self, tokens) -> str:
        """backend.rs:98-121: Hugging Face decodes; SentencePiece joins the pieces encode has seen
        and fails when one is missing."""
        if self._backend == "hf":
            return self._inner.decode([int(t) for t in tokens], skip_special_tokens=False)
        pieces = [self._id_to_piece[int(t)] for t in tokens if int(t) in self._id_to_piece]
        if len(pieces) != len(tokens):
            raise TokenizerError(f"cannot decode: missing piece strings for {len(tokens) - len(pieces)} out of "
                                 f"{len(tokens)} tokens (decode needs cache from encode)")
        return "".join(pieces)

    def vocab_size(self) -> int:
        """backend.rs:123-128 (0 for SentencePiece, as the reference reports)."""
        return self._inner.get_vocab_size(True) if self._backend == "hf" else 0


# ---- prompt styles (src/chat_prompt.rs) --------------------------------------------------------

GEMMA4_E2B_ASSISTANT_STOP_MARKERS = ("<turn|>", "<turn|", "<|turn>", "<|turn", "<|tool_call", "<|tool_response",
                                     "<|tool>", "<tool|>", "<|tool", "<|audio", "<|image", "<|video")


def gemma4_e2b_strip_thinking_blocks(s: str) -> str:
    """Drop `<|channel>` ... `<channel|>` blocks; an unterminated one drops the rest
    (chat_prompt.rs:29-53)."""
    start_m, end_m = "<|channel>", "<channel|>"
    out, rest = [], s
    while True:
        start = rest.find(start_m)
        if start < 0:
            out.append(rest)
            break
        out.append(rest[:start])
        after = rest[start + len(start_m):]
        end = after.find(end_m)
        if end < 0:
            break
        rest = after[end + len(end_m):]
    return "".join(out)


def gemma4_e2b_truncate_assistant_at_structure(s: str) -> str:
    """Cut before the first structure / modality marker (chat_prompt.rs:56-65)."""
    end = len(s)
    for m in GEMMA4_E2B_ASSISTANT_STOP_MARKERS:
        i = s.find(m)
        if i >= 0:
            end = min(end, i)
    return s[:end]


def gemma4_e2b_decode_has_structure_marker(s: str) -> bool:
    return len(gemma4_e2b_truncate_assistant_at_structure(s)) < len(s)


def gemma4_e2b_strip_dangling_contraction_tail(s: str) -> str:
    """Drop a trailing single ASCII letter + apostrophe word (chat_prompt.rs:75-92)."""
    s = s.rstrip()
    if not s.endswith("'"):
        return s
    no_quote = s[:-1].rstrip()
    ws = [i for i, c in enumerate(no_quote) if c.isspace()]
    tail_start = ws[-1] + 1 if ws else 0
    tail = no_quote[tail_start:]
    if len(tail) == 1 and tail.isascii() and tail.isalpha():
        return no_quote[:tail_start].rstrip()
    return s


def gemma4_e2b_assistant_visible(s: str) -> str:
    """Truncate at markers, then tidy a partial contraction only if a marker was present
    (chat_prompt.rs:95-105)."""
    no_think = gemma4_e2b_strip_thinking_blocks(s)
    had_marker = gemma4_e2b_decode_has_structure_marker(no_think)
    t = gemma4_e2b_truncate_assistant_at_structure(no_think)
    if had_marker:
        t = gemma4_e2b_strip_dangling_contraction_tail(t)
    return t.rstrip()


class ChatPromptStyle(Enum):
    """ChatPromptStyle (chat_prompt.rs:137-200)."""
    RAW = "raw"
    MISTRAL_INSTRUCT = "mistral-instruct"
    GEMMA4_E2B = "gemma4-e2b"

    @classmethod
    def parse(cls, s: str) -> "ChatPromptStyle | None":
        v = s.strip().lower()
        if v in ("", "raw", "none"):
            return cls.RAW
        if v in ("mistral", "mistral-instruct", "instruct"):
            return cls.MISTRAL_INSTRUCT
        if v in ("gemma", "gemma4", "gemma4-e2b", "gemma-e2b"):
            return cls.GEMMA4_E2B
        return None

    def wrap(self, user: str) -> str:
        """Single turn (chat_prompt.rs:164-176)."""
        user = user.strip()
        if self is ChatPromptStyle.RAW:
            return user
        if self is ChatPromptStyle.MISTRAL_INSTRUCT:
            return f"[INST] {user} [/INST]"
        return f"<|turn>user\n{user}<turn|>\n<|turn>model\n"


# ---- generation (src/main.rs:84-126) -------------------------------------------------------------

def generate(model: "E.LoadedModel", tokenizer: Tokenizer, prompt: str, new_tokens: int = 20,
             chat: ChatPromptStyle = ChatPromptStyle.RAW, temperature: float = 0.0, rng=None,
             session: "E.InferenceSession | None" = None) -> tuple[str, list[int]]:
    """The CLI's loop: wrap the prompt for its style, encode with the model's BOS/EOS rule,
    prefill, then up to `new_tokens` x { next id (greedy on the device, or sample_temperature on
    the device when temperature > 0, drawing r from `rng`); stop at EOS; stop at a Gemma structure
    marker; decode it }. Returns (visible continuation, generated ids)."""
    text = chat.wrap(prompt)
    cfg = TokenizerPromptConfig.from_model(model)
    ids = tokenizer.encode_with_prompt_config(text, cfg)
    s = session or E.InferenceSession(model)
    s.reset()
    s.prefill(ids)
    generated: list[int] = []
    for _ in range(new_tokens):
        if temperature > 0.0:
            nxt = E.sample_temperature_next_token(s, temperature, float(rng.random()))
        else:
            nxt = E.greedy_next_token(s)
        if nxt == cfg.eos_token_id:
            break
        generated.append(nxt)
        if chat is ChatPromptStyle.GEMMA4_E2B and gemma4_e2b_decode_has_structure_marker(
                tokenizer.decode_piece_ids(generated)):
            break
        s.decode_token(nxt)
    raw = tokenizer.decode_piece_ids(generated)
    visible = gemma4_e2b_assistant_visible(raw) if chat is ChatPromptStyle.GEMMA4_E2B else raw.rstrip()
    return visible, generated


def main(argv=None) -> int:
    """src/main.rs: greedy continuation of PROMPT (or one line of stdin), printed on stdout.
    Errors print the message and return 1."""
    ap = argparse.ArgumentParser(prog="python -m inference_engine_rust_amd",
                                 description="Greedy LM generation (GGUF + tokenizer .model or .json)")
    ap.add_argument("-m", "--model", default="model/mistral-7b-v0.1/mistral-7b-v0.1.Q4_K_M.gguf",
                    help="GGUF model path")
    ap.add_argument("-t", "--tokenizer", default="model/mistral-7b-v0.1/tokenizer.model",
                    help="SentencePiece tokenizer.model or Hugging Face tokenizer.json")
    ap.add_argument("-n", "--new-tokens", type=int, default=20, help="how many new tokens to append")
    ap.add_argument("--chat", default="raw", help="prompt style: raw | mistral-instruct | gemma4-e2b")
    ap.add_argument("--temperature", type=float, default=0.0,
                    help="> 0: sample_temperature on the device instead of greedy (not in the reference CLI)")
    ap.add_argument("--seed", type=int, default=0, help="seed of the uniform draws when sampling")
    ap.add_argument("prompt", nargs="?", default=None, help="prompt text; one line of stdin when omitted")
    a = ap.parse_args(argv)
    try:
        if a.prompt is not None:
            if not a.prompt.strip():
                raise E.EngineError(_ERR_MODEL, "prompt is empty")
            prompt = a.prompt
        else:
            prompt = sys.stdin.readline().rstrip("\r\n")
        if not prompt:
            raise E.EngineError(_ERR_MODEL, "no prompt: pass PROMPT or pipe a line on stdin")
        style = ChatPromptStyle.parse(a.chat)
        if style is None:
            raise E.EngineError(_ERR_MODEL, f"unknown --chat {a.chat!r}: use raw | mistral-instruct | gemma4-e2b")
        if not os.path.isfile(a.tokenizer):
            raise E.EngineError(_ERR_MODEL, f"tokenizer file not found: {a.tokenizer}")
        model = E.LoadedModel.load(a.model)
        tok = Tokenizer.load_from_file(a.tokenizer)
        import random
        text, _ = generate(model, tok, prompt, a.new_tokens, style, a.temperature, random.Random(a.seed))
    except (E.EngineError, TokenizerError) as e:
        print(f"error: {e}", file=sys.stderr)
        return 1
    print(text)
    return 0
