"""Qwen2-VL adapter: model-specific pieces the generic runner delegates to.

Mirrors the ``VLMAdapter`` interface (omniserve/models/base.py:24-74) as implemented
by ``Qwen2VLAdapter`` (models/qwen2_vl.py:30-122) for the text decoder:
embed_tokens (:93-94), prefill_positions (:100-106), decode_positions (:108-112),
llm (:115-116), plus the shape attributes the KV pool needs.

Weights (models/qwen2_vl.py:31-61): ``quant="gptq"`` with ``gptq_dir`` reads the
AutoGPTQ checkpoint's decoder tensors, ``quant=None`` with ``model_dir`` the fp16
Hugging Face checkpoint's (``checkpoint``); without a directory (the reference would
look in its default cache paths, which do not exist offline) seeded synthetic weights
of the real architecture are built (``synth``); ``weights=`` accepts an already built
dict (fp16 or GPTQ layout).  ``quant="gptq"`` selects the int4 path (every decoder
linear W4A16, embeddings / lm_head fp16, as kernels/marlin_linear.py:114-143);
``"marlin"`` quantises the fp16 MLP linears to int4 by rounding (no calibration) and
``"mixed"`` applies the default per-op plan (gate_up and down FP8 W8A8, attention
projections fp16), as models/qwen2_vl.py:56-64 do.
"""

from __future__ import annotations

from typing import List, Optional

import torch

from . import synth
from .positions import IMAGE_TOKEN_ID, mrope_positions
from .qwen2_llm import Qwen2LLM

EOS_ID = 151645  # <|im_end|>


class Qwen2VLAdapter:
    def __init__(self, model_dir: Optional[str] = None, quant: Optional[str] = None,
                 gptq_dir: Optional[str] = None, weights: Optional[dict] = None,
                 shape: Optional[synth.DecoderShape] = None, seed: int = 0,
                 num_layers: Optional[int] = None, device="cuda", max_pos: int = 8192,
                 vision=None):
        if not self.supports_quant(quant):
            raise ValueError(f"unsupported quant {quant!r} (None, 'marlin', 'gptq' or 'mixed')")
        self.device = torch.device(device)
        self.shape = shape or synth.DecoderShape()
        if num_layers is not None:
            self.shape.num_layers = num_layers
        self.quant = quant
        src = gptq_dir if quant == "gptq" else model_dir
        vision_sd = vision if isinstance(vision, dict) else None
        if weights is None and src is not None:
            from . import checkpoint
            sd = checkpoint.read_safetensors(src)
            weights = (checkpoint.gptq_decoder_from_state_dict(sd) if quant == "gptq"
                       else checkpoint.fp16_decoder_from_state_dict(sd))
            if vision_sd is None:
                vision_sd = checkpoint.vision_state_dict(sd)
            del sd
            if weights["embed"].shape[1] != self.shape.hidden_size:
                raise ValueError(f"checkpoint hidden size {weights['embed'].shape[1]} is not the "
                                 f"Qwen2-VL-2B decoder's {self.shape.hidden_size}")
            self.shape.num_layers = len(weights["layers"])
            self.shape.vocab_size = weights["embed"].shape[0]
        if weights is None:
            gen = synth.gptq_decoder if quant == "gptq" else synth.fp16_decoder
            weights = gen(self.shape, seed=seed)
        build = Qwen2LLM.from_gptq if quant == "gptq" else Qwen2LLM.from_fp16
        self._llm = build(weights, self.shape, self.device, max_pos=max_pos)
        # models/qwen2_vl.py:56-64: RTN int4 MLP, or the per-op mixed-precision plan
        if quant == "marlin":
            from .mixed_precision import quantize_llm_marlin
            quantize_llm_marlin(self._llm, scope="mlp")
        elif quant == "mixed":
            from .mixed_precision import apply_mixed
            apply_mixed(self._llm)
        # vision tower (models/qwen2_vl.py:46-48): the checkpoint's visual.* tensors, a
        # given state dict, or (vision=True / an int depth) seeded synthetic weights
        self._vit = None
        if vision_sd is None and vision is not None and vision is not False:
            from .vit import VisionConfig
            depth = None if vision is True else int(vision)
            vision_sd = synth.vision_tower(VisionConfig(), seed=seed, depth=depth)
        if vision_sd:
            from .vit import Qwen2VIT, load_vit_from_state_dict
            depth = sum(1 for k in vision_sd if k.startswith("visual.blocks.") and
                        k.endswith(".norm1.weight"))
            self._vit = load_vit_from_state_dict(Qwen2VIT(depth=depth, device=self.device),
                                                 vision_sd)
        self.num_layers = len(weights["layers"])
        self.num_kv_heads = self.shape.num_kv_heads
        self.num_heads = self.shape.num_heads
        self.head_dim = self.shape.head_dim
        self.image_token_id = IMAGE_TOKEN_ID
        self.eos_ids = {EOS_ID}

    @property
    def model(self) -> Qwen2LLM:
        return self._llm

    # ---- input side ---------------------------------------------------------------
    def encode_prompt(self, prompt, grids=None) -> List[int]:
        """Token ids of a prompt: a list of ids is taken as is; a string must be
        whitespace-separated integer ids (there is no tokenizer offline)."""
        if isinstance(prompt, str):
            return list(map(int, prompt.split()))
        return list(map(int, prompt))

    def embed_tokens(self, input_ids: torch.Tensor) -> torch.Tensor:
        return self._llm.embed_tokens(input_ids)

    @property
    def vision(self):
        """The vision tower (None when the adapter was built without one)."""
        return self._vit

    def vision_embed(self, images) -> torch.Tensor:
        """Concatenated vision rows of the request's images, in order
        (models/qwen2_vl.py:96-97): ``PixelInput`` items go through the vision tower in one
        call (their cu_seqlens keep the images apart), ``VisionInput`` rows are taken as
        given."""
        from .request import PixelInput
        pix = [im for im in images if isinstance(im, PixelInput)]
        enc = []
        if pix:
            if self._vit is None:
                raise RuntimeError("pixel inputs need the vision tower: build the adapter from "
                                   "a checkpoint with visual.* tensors, or with vision=True")
            pv = torch.cat([torch.as_tensor(im.pixel_values).to(self.device, torch.float16)
                            for im in pix], 0)
            out = self._vit(pv, [im.grid for im in pix])
            sizes = [im.grid[0] * im.grid[1] * im.grid[2] // 4 for im in pix]
            enc = list(torch.split(out, sizes, 0))
        rows = []
        for im in images:
            rows.append(enc.pop(0) if isinstance(im, PixelInput)
                        else im.embeds.to(self.device, torch.float16))
        return torch.cat(rows, 0)

    # ---- positions (M-RoPE) -------------------------------------------------------
    def prefill_positions(self, input_ids, grids):
        L = len(input_ids)
        if not grids:
            pos = torch.arange(L, dtype=torch.int64).view(1, -1).expand(3, -1)
            return pos, 0
        return mrope_positions(input_ids, grids, self.image_token_id)

    def decode_positions(self, write_pos: torch.Tensor, rope_deltas: torch.Tensor):
        n = write_pos.shape[0]
        pos = torch.empty(3, n, 1, device=write_pos.device, dtype=torch.long)
        pos[:, :, 0] = (write_pos + rope_deltas).unsqueeze(0)
        return pos

    # ---- forward ------------------------------------------------------------------
    def llm(self, embeds, positions, attn_mask, cache, logits_indices=None):
        return self._llm(embeds, positions, attn_mask, cache, logits_indices=logits_indices)

    def detokenize(self, token_ids) -> str:
        return " ".join(str(int(t)) for t in token_ids)

    @staticmethod
    def supports_quant(quant) -> bool:
        return quant in (None, "marlin", "gptq", "mixed")
