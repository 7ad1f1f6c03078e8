"""Writes tests/golden/vae_decoder_layout.json: the names, dtypes and shapes of the VAE decoder's
tensors in the pinned checkpoint, taken from the reference's published layout file
(configs/checkpoint-layout.json, read by HTTP range request from the pinned revision by the
reference's scripts/verify_checkpoint_layout.py). Only the tensors the decoder reads are kept
(post_quant_conv.* and decoder.*). Data only: the reference is read as JSON, nothing of it runs.

    python tests/golden/make_vae_layout.py [/root/reference]
"""
import json
import sys
from pathlib import Path

ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
layout = json.loads((ref / "configs" / "checkpoint-layout.json").read_text())
keep = {k: v for k, v in sorted(layout["tensors"].items())
        if k.startswith("decoder.") or k.startswith("post_quant_conv.")}
out = {"_what": "VAE decoder tensors of the pinned checkpoint (names, dtypes, shapes), extracted "
                "from the reference's configs/checkpoint-layout.json by make_vae_layout.py",
       "source": layout["sources"]["vae/diffusion_pytorch_model.safetensors"], "tensors": keep}
Path(__file__).with_name("vae_decoder_layout.json").write_text(json.dumps(out, indent=1) + "\n")
print(f"{len(keep)} tensors")
