"""Caller-side request state the runner reads and writes.

Same fields and behaviour as omniserve/request.py (Status :21-25, SamplingParams
:28-37, Request :40-47, Sequence :50-115), so a scheduler/engine written against
the reference drives this runner unchanged.  ``Request.images`` holds, per image,
either ``PixelInput`` (the image processor's flattened patches + grid, encoded by the
adapter's vision tower, as models/qwen2_vl.py:76-97 does) or ``VisionInput``
(precomputed vision rows + grid: the tower's output, supplied by the caller).
"""

from __future__ import annotations

import enum
import itertools
import time
from dataclasses import dataclass, field
from typing import List, Optional, Tuple

_counter = itertools.count()


class Status(enum.Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"
    ABORTED = "aborted"


@dataclass
class SamplingParams:
    max_new_tokens: int = 128
    temperature: float = 0.0          # 0 -> greedy
    top_p: float = 1.0
    stop_token_ids: List[int] = field(default_factory=list)

    @property
    def greedy(self) -> bool:
        return self.temperature == 0.0


@dataclass
class VisionInput:
    """Vision-embedding rows [n_tokens, hidden] fp16 for one image and its patch grid
    (t, h, w) before the 2x2 merge, as the reference's ViT + merger would produce."""
    embeds: object
    grid: Tuple[int, int, int]


@dataclass
class PixelInput:
    """One image as the vision tower takes it: normalised pixel patches fp16
    [t*h*w, 3*2*14*14] in merge-window order (the reference's preprocess_image output,
    model/preprocess.py) and the patch grid (t, h, w); it becomes t*h*w/4 rows."""
    pixel_values: object
    grid: Tuple[int, int, int]


@dataclass
class Request:
    prompt: object                     # str, or a list of token ids
    images: List[VisionInput] = field(default_factory=list)
    sampling: SamplingParams = field(default_factory=SamplingParams)
    request_id: str = field(default_factory=lambda: f"req-{next(_counter)}")
    arrival_t: float = field(default_factory=time.perf_counter)


@dataclass
class Sequence:
    request: Request
    prompt_token_ids: List[int] = field(default_factory=list)
    output_token_ids: List[int] = field(default_factory=list)
    status: Status = Status.WAITING
    kv_handle: Optional[dict] = None   # {"slot": int, "rope_delta": int}
    vision_embeds: Optional[object] = None
    num_prefilled: int = 0
    prefill_chunk: int = 0
    num_streamed: int = 0
    first_token_t: Optional[float] = None
    finish_t: Optional[float] = None

    @property
    def request_id(self) -> str:
        return self.request.request_id

    @property
    def num_prompt_tokens(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def num_output_tokens(self) -> int:
        return len(self.output_token_ids)

    @property
    def total_len(self) -> int:
        return self.num_prompt_tokens + self.num_output_tokens

    def last_token_id(self) -> int:
        return self.output_token_ids[-1] if self.output_token_ids else self.prompt_token_ids[-1]

    def append_token(self, token_id: int) -> None:
        if self.first_token_t is None:
            self.first_token_t = time.perf_counter()
        self.output_token_ids.append(token_id)

    def maybe_finish(self) -> bool:
        sp = self.request.sampling
        if self.output_token_ids and self.output_token_ids[-1] in sp.stop_token_ids:
            self._finish()
            return True
        if self.num_output_tokens >= sp.max_new_tokens:
            self._finish()
            return True
        return False

    def _finish(self) -> None:
        self.status = Status.FINISHED
        self.finish_t = time.perf_counter()
