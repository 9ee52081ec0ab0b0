"""M-RoPE 3-D position ids for text + images (omniserve/model/positions.py:17-58).

Text tokens take sequential positions on all three (t, h, w) axes; an image run of
t * (h/2) * (w/2) tokens takes its merged-grid coordinates offset by the text
before it; text after an image resumes at max + 1.  Returns the ids and the
per-sequence ``rope_delta = max + 1 - L`` that decode adds to the write position
(models/qwen2_vl.py:100-112).  Vectorised with numpy (no per-token Python loop).
"""

from __future__ import annotations

import functools
from typing import Sequence, Tuple

import numpy as np
import torch

IMAGE_TOKEN_ID = 151655
VISION_START_TOKEN_ID = 151652
SPATIAL_MERGE_SIZE = 2


@functools.lru_cache(maxsize=64)
def _grid_offsets(t: int, gh: int, gw: int) -> Tuple[np.ndarray, int]:
    """(t, h, w) offsets [3, t gh gw] of a merged image grid's tokens in row-major order,
    and their largest value (read-only; cached per grid shape)."""
    n = t * gh * gw
    if n == 0:
        raise ValueError("empty image grid")
    off = np.empty((3, n), dtype=np.int64)
    off[0] = np.repeat(np.arange(t), gh * gw)
    off[1] = np.tile(np.repeat(np.arange(gh), gw), t)
    off[2] = np.tile(np.arange(gw), t * gh)
    off.setflags(write=False)
    return off, max(t, gh, gw) - 1


def mrope_positions(input_ids: Sequence[int], grids: Sequence[Tuple[int, int, int]],
                    image_token_id: int = IMAGE_TOKEN_ID,
                    vision_start_id: int = VISION_START_TOKEN_ID,
                    merge: int = SPATIAL_MERGE_SIZE) -> Tuple[torch.Tensor, int]:
    """(pos [3, L] int64, rope_delta) of one prompt.  As in positions.py:27-30 the number of
    images is the number of vision-start tokens directly followed by an image token; image i
    is the run at the first image token at or after the current index (:35) and takes
    grids[i]; every piece starts at the previous piece's max + 1, so the largest position is
    the last piece's and rope_delta = that + 1 - L."""
    ids = np.asarray(input_ids, dtype=np.int64)
    L = ids.shape[0]
    pos = np.empty((3, L), dtype=np.int64)
    vs = np.flatnonzero(ids[:-1] == vision_start_id) if L > 1 else np.empty(0, np.int64)
    n_images = int(np.count_nonzero(ids[vs + 1] == image_token_id)) if vs.size else 0
    if n_images > len(grids):
        raise ValueError(f"{n_images} images in the prompt, {len(grids)} grids given")
    img_at = np.flatnonzero(ids == image_token_id) if n_images else None
    st = 0          # next token index
    nxt = 0         # next position value (previous piece's max + 1)
    for (t, h, w) in list(grids)[:n_images]:
        ed = int(img_at[np.searchsorted(img_at, st)])
        off, omax = _grid_offsets(int(t), int(h) // merge, int(w) // merge)
        n_img = off.shape[1]
        if ed + n_img > L:
            raise ValueError("image grid longer than the prompt's image run")
        text_len = ed - st
        pos[:, st:ed] = np.arange(nxt, nxt + text_len)
        base = nxt + text_len
        np.add(off, base, out=pos[:, ed:ed + n_img])
        nxt = base + omax + 1
        st = ed + n_img
    if st < L:
        pos[:, st:] = np.arange(nxt, nxt + L - st)
        nxt += L - st
    delta = nxt - L if L else 0
    return torch.from_numpy(pos), delta
