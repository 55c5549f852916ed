"""Python API over the C ABI, mirroring the reference's PyO3 `BitNet` class
(oxbitnet-python/src/lib.rs:26-213, python/oxbitnet/__init__.pyi).

    bn = BitNet.load_sync("model.gguf")
    bn.generate("Hello", print, max_tokens=32)
    text = bn.generate_sync("Hello", max_tokens=32)
    bn.dispose()

Like the reference binding, `repeat_last_n` is fixed at 64 (make_options,
lib.rs:11-24).  Additionally `Model` exposes the ids-level engine
(forward / greedy decode) used by the parity tests and the benchmark.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._native import (ChatMessage, GenerateOptions, LoadOptions, ModelInfo, NativeError,
                      ProgressFn, TokenFn, check, last_error, lib)


def _ref_error() -> str:
    msg = lib().oxbitnet_error_message()
    return msg.decode() if msg else "unknown error"


class BitNet:
    def __init__(self, handle: int):
        self._h = handle

    @staticmethod
    def load_sync(source: str, on_progress=None) -> "BitNet":
        opts = lib().oxbitnet_default_load_options()
        cb = None
        if on_progress is not None:
            cb = ProgressFn(lambda p, ud: on_progress(p.contents.phase, p.contents.loaded,
                                                      p.contents.total, p.contents.fraction))
            opts.on_progress = cb
        h = lib().oxbitnet_load(source.encode(), C.byref(opts))
        if not h:
            raise RuntimeError(_ref_error())
        return BitNet(h)

    def _opts(self, max_tokens, temperature, top_k, repeat_penalty) -> GenerateOptions:
        o = lib().oxbitnet_default_generate_options()
        o.max_tokens, o.temperature, o.top_k = max_tokens, temperature, top_k
        o.repeat_penalty, o.repeat_last_n = repeat_penalty, 64
        return o

    def _live(self):
        if not self._h:
            raise RuntimeError("Model disposed")
        return self._h

    def generate(self, prompt: str, on_token, max_tokens: int = 256, temperature: float = 1.0,
                 top_k: int = 50, repeat_penalty: float = 1.1) -> int:
        count = [0]

        def cb(tok, n, ud):
            count[0] += 1
            on_token(C.string_at(tok, n).decode("utf-8", "replace"))
            return 0

        fn = TokenFn(cb)
        o = self._opts(max_tokens, temperature, top_k, repeat_penalty)
        if lib().oxbitnet_generate(self._live(), prompt.encode(), C.byref(o), fn, None) != 0:
            raise RuntimeError(_ref_error())
        return count[0]

    def chat(self, messages, on_token, max_tokens: int = 256, temperature: float = 1.0,
             top_k: int = 50, repeat_penalty: float = 1.1) -> int:
        keep = [(r.encode(), c.encode()) for r, c in messages]
        arr = (ChatMessage * len(keep))(*[ChatMessage(r, c) for r, c in keep])
        count = [0]

        def cb(tok, n, ud):
            count[0] += 1
            on_token(C.string_at(tok, n).decode("utf-8", "replace"))
            return 0

        fn = TokenFn(cb)
        o = self._opts(max_tokens, temperature, top_k, repeat_penalty)
        if lib().oxbitnet_chat(self._live(), arr, len(keep), C.byref(o), fn, None) != 0:
            raise RuntimeError(_ref_error())
        return count[0]

    def generate_tokens_sync(self, prompt: str, max_tokens: int = 256, temperature: float = 1.0,
                             top_k: int = 50) -> list[str]:
        out: list[str] = []
        self.generate(prompt, out.append, max_tokens, temperature, top_k, 1.1)
        return out

    def generate_sync(self, prompt: str, max_tokens: int = 256, temperature: float = 1.0,
                      top_k: int = 50) -> str:
        return "".join(self.generate_tokens_sync(prompt, max_tokens, temperature, top_k))

    def dispose(self) -> None:
        if self._h:
            lib().oxbitnet_free(self._h)
            self._h = None

    def __repr__(self) -> str:
        return "BitNet(loaded)" if self._h else "BitNet(disposed)"

    def __del__(self):
        try:
            self.dispose()
        except Exception:
            pass


class Model:
    """ids-level engine (include/oxbitnet_ops.h oxb_model_*)."""

    def __init__(self, path: str, max_seq: int = 4096, kv: str = "f16"):
        """kv: the KV cache type, "f16" (throughput) or "f32" (the reference's)."""
        if kv not in ("f16", "f32"):
            raise ValueError(f"kv must be 'f16' or 'f32', not {kv!r}")
        self._m = lib().oxb_model_load_kv(path.encode(), max_seq, int(kv == "f32"))
        if not self._m:
            raise NativeError(last_error())
        info = ModelInfo()
        check(lib().oxb_model_get_info(self._m, C.byref(info)), "model info")
        self.info = {k: getattr(info, k) for k, _ in ModelInfo._fields_}

    @property
    def vocab(self) -> int:
        return self.info["vocab"]

    def reset(self) -> None:
        check(lib().oxb_model_reset(self._m), "reset")

    @property
    def position(self) -> int:
        return lib().oxb_model_position(self._m)

    def forward(self, ids, want_logits: bool = True):
        """forward(ids) at the current position -> (greedy token, logits or None)."""
        ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
        logits = np.empty(self.vocab, np.float32) if want_logits else None
        tok = lib().oxb_model_forward(self._m, ids.ctypes.data, ids.size,
                                      logits.ctypes.data if want_logits else None)
        if tok < 0:
            raise NativeError(last_error())
        return tok, logits

    def decode_greedy(self, n_steps: int) -> np.ndarray:
        out = np.empty(n_steps, np.int32)
        check(lib().oxb_model_decode_greedy(self._m, n_steps, out.ctypes.data), "decode")
        return out

    def set_token(self, tok: int) -> None:
        check(lib().oxb_model_set_token(self._m, int(tok)), "set_token")

    def step(self, want_logits: bool = True):
        logits = np.empty(self.vocab, np.float32) if want_logits else None
        tok = lib().oxb_model_step(self._m, logits.ctypes.data if want_logits else None)
        if tok < 0:
            raise NativeError(last_error())
        return tok, logits

    def set_sampling(self, u=None, temperature: float = 1.0, top_k: int = 50,
                     repeat_penalty: float = 1.1, repeat_last_n: int = 64) -> None:
        """Draw the tokens of later forwards / steps on the device
        (oxb_model_set_sampling); u[i] is the uniform draw of the i-th token
        since reset.  u=None: back to the LM head's argmax."""
        if u is None:
            check(lib().oxb_model_set_sampling(self._m, 1.0, 0, 1.0, 0, None, 0), "sampling")
            return
        u = np.ascontiguousarray(u, np.float32).reshape(-1)
        check(lib().oxb_model_set_sampling(self._m, float(temperature), int(top_k),
                                           float(repeat_penalty), int(repeat_last_n),
                                           u.ctypes.data, u.size), "sampling")

    def close(self) -> None:
        if self._m:
            lib().oxb_model_free(self._m)
            self._m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Batch:
    """Batched greedy decode of independent sequences on a loaded Model
    (include/oxbitnet_ops.h oxb_batch_*); each slot's tokens and logits are
    those of a one-sequence Model on the same prompt."""

    def __init__(self, model: Model, batch: int, max_seq: int):
        self._model = model   # keeps the weights alive
        self._b = lib().oxb_batch_create(model._m, batch, max_seq)
        if not self._b:
            raise NativeError(last_error())
        self.batch = batch

    def prefill(self, slot: int, ids) -> int:
        ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
        tok = lib().oxb_batch_prefill(self._b, slot, ids.ctypes.data, ids.size)
        if tok < 0:
            raise NativeError(last_error())
        return tok

    def decode_greedy(self, n_steps: int) -> np.ndarray:
        out = np.empty((self.batch, n_steps), np.int32)
        check(lib().oxb_batch_decode_greedy(self._b, n_steps, out.ctypes.data), "batch decode")
        return out

    def position(self, slot: int) -> int:
        return lib().oxb_batch_position(self._b, slot)

    def logits(self) -> np.ndarray:
        out = np.empty((self.batch, self._model.vocab), np.float32)
        check(lib().oxb_batch_logits(self._b, out.ctypes.data), "batch logits")
        return out

    def close(self) -> None:
        if self._b:
            lib().oxb_batch_free(self._b)
            self._b = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
