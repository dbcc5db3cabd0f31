"""Streamed text of one sequence: incremental detokenization and stop strings.

The contract is the engine's ``_TextStream`` (src/vinfer/runtime/generate.py:27-88), kept so a
request streams the same text whether the engine's one-sequence loop or the batched loop here
produced its tokens:

- each push decodes only a short window of recent tokens: the text the window's new tokens add
  is the decode of the whole window minus the decode of its older part, so context-dependent
  spacing is kept and the cost per token does not grow with the output;
- a window whose decode ends in U+FFFD (an unfinished UTF-8 sequence) waits for more tokens,
  and so does one whose new tokens rewrote earlier text, until it settles;
- text that may still turn into a stop string is held back (the longest stop string's length
  minus one characters), so streamed text is never taken back; on a stop string the text ends
  just before it.
"""

from __future__ import annotations

from collections.abc import Callable

_UNFINISHED = "�"


class TextStream:
    def __init__(self, decode: Callable[[list[int]], str], stops: tuple[str, ...] = ()) -> None:
        self._decode = decode
        self._stops = tuple(s for s in stops if s)
        self._hold = max(map(len, self._stops), default=1) - 1  # characters held back
        self._tokens: list[int] = []
        self._start = 0  # window start: tokens before it are settled in self._text
        self._seen = 0  # tokens [start, seen) were in the window at the last settled decode
        self._text = ""  # text of every settled token
        self._out = 0  # characters of self._text already returned

    @property
    def text(self) -> str:
        """The text decoded so far (emitted or held back)."""
        return self._text

    def _settle(self, final: bool) -> None:
        window = self._tokens[self._start :]
        old = self._decode(window[: self._seen - self._start])
        new = self._decode(window)
        if not final and new.endswith(_UNFINISHED):
            return  # wait for the rest of the character
        if len(new) <= len(old) and new != old:
            return  # the new tokens rewrote earlier text: wait until the window settles
        self._text += new[len(old) :]
        # Slide the window even when no text was added (a token that decodes to nothing), so it
        # stays a few tokens long.
        self._start, self._seen = self._seen, len(self._tokens)

    def push(self, token_id: int | None) -> tuple[str, bool]:
        """Add one token (``None``: none, the final flush). Returns ``(new text, stop hit)``."""
        final = token_id is None
        if not final:
            self._tokens.append(token_id)
        self._settle(final)
        text = self._text
        lo = max(0, self._out - self._hold)
        found = [i for i in (text.find(s, lo) for s in self._stops) if i >= 0]
        if found:
            cut = min(found)
            piece = text[self._out : cut]
            self._out = max(self._out, cut)
            return piece, True
        end = len(text) if final else len(text) - self._hold
        if end <= self._out:
            return "", False
        piece, self._out = text[self._out : end], end
        return piece, False

    def flush(self) -> str:
        """Everything held back, up to a stop string if one is found."""
        return self.push(None)[0]
