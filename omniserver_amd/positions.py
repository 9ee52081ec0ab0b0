"""M-RoPE 3-D position ids for text + images (omniserve/model/positions.py:17-58).

Text tokens take sequential positions on all three (t, h, w) axes; an image run of
t * (h/2) * (w/2) tokens takes its merged-grid coordinates offset by the text
before it; text after an image resumes at max + 1.  Returns the ids and the
per-sequence ``rope_delta = max + 1 - L`` that decode adds to the write position
(models/qwen2_vl.py:100-112).  Vectorised with numpy (no per-token Python loop).
"""

from __future__ import annotations

from typing import Sequence, Tuple

import numpy as np
import torch

IMAGE_TOKEN_ID = 151655
VISION_START_TOKEN_ID = 151652
SPATIAL_MERGE_SIZE = 2


def mrope_positions(input_ids: Sequence[int], grids: Sequence[Tuple[int, int, int]],
                    image_token_id: int = IMAGE_TOKEN_ID,
                    merge: int = SPATIAL_MERGE_SIZE) -> Tuple[torch.Tensor, int]:
    ids = np.asarray(input_ids, dtype=np.int64)
    L = ids.shape[0]
    pos = np.empty((3, L), dtype=np.int64)
    st = 0          # next token index
    nxt = 0         # next position value
    img_at = np.flatnonzero(ids == image_token_id)
    for (t, h, w) in grids:
        later = img_at[img_at >= st]
        if later.size == 0:
            raise ValueError("more image grids than image token runs")
        ed = int(later[0])
        gh, gw = h // merge, w // merge
        n_img = t * gh * gw
        text_len = ed - st
        pos[:, st:ed] = np.arange(text_len) + nxt
        base = nxt + text_len
        pos[0, ed:ed + n_img] = np.repeat(np.arange(t), gh * gw) + base
        pos[1, ed:ed + n_img] = np.tile(np.repeat(np.arange(gh), gw), t) + base
        pos[2, ed:ed + n_img] = np.tile(np.arange(gw), t * gh) + base
        nxt = int(pos[:, ed:ed + n_img].max()) + 1
        st = ed + n_img
    if st < L:
        pos[:, st:] = np.arange(L - st) + nxt
    delta = int(pos.max()) + 1 - L if L else 0
    return torch.from_numpy(pos), delta
