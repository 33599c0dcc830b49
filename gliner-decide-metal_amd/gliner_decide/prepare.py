"""The weight step of Tools/prepare_model.py:82-113, on a checkpoint already
on disk: keep the `encoder.*` and `classifier.*` tensors of the upstream
GLiNER2.5-Decide model.safetensors, cast floating-point tensors to fp16,
require the tensors the classifier cannot run without, and write
decide-classification-fp16.safetensors with the same metadata.

    python -m gliner_decide.prepare --source model.safetensors --output Artifacts
        [--encoder-config encoder_config/config.json]

Fetching the checkpoint (`hf_hub_download`, :73-80) and the Core ML runtime
(:115-130) needs the network and is left to the caller; `--encoder-config`
copies the encoder's config.json beside the weights as encoder-config.json.
"""

from __future__ import annotations

import argparse
import shutil
import sys
from pathlib import Path

import numpy as np

SOURCE_MODEL = "fastino/GLiNER2.5-Decide"
SOURCE_REVISION = "65624f1a0265b3f612bae66a2685a06b94a68a9d"
REQUIRED = ("encoder.embeddings.word_embeddings.weight", "encoder.encoder.rel_embeddings.weight",
            "encoder.encoder.LayerNorm.weight", "classifier.0.weight", "classifier.2.weight")
OUTPUT_NAME = "decide-classification-fp16.safetensors"


def prepare_weights(source: str | Path, output_dir: str | Path, encoder_config: str | Path | None = None,
                    source_model: str = SOURCE_MODEL, source_revision: str = SOURCE_REVISION) -> Path:
    """prepare_model.py:82-113 without the download; returns the written path."""
    import torch
    from safetensors import safe_open
    from safetensors.numpy import save_file
    source, out = Path(source), Path(output_dir)
    converted = {}
    # read through torch: it also holds bf16 tensors, which numpy cannot;
    # its fp32 -> fp16 cast rounds to nearest even, as numpy's astype does
    with safe_open(str(source), framework="pt", device="cpu") as f:
        for key in f.keys():
            if not (key.startswith("encoder.") or key.startswith("classifier.")):
                continue
            t = f.get_tensor(key)
            if t.is_floating_point():
                t = t.to(torch.float16)
            converted[key] = np.ascontiguousarray(t.numpy())
    missing = sorted(set(REQUIRED).difference(converted))
    if missing:
        raise RuntimeError(f"Checkpoint is missing required weights: {missing}")
    out.mkdir(parents=True, exist_ok=True)
    path = out / OUTPUT_NAME
    save_file(converted, str(path), metadata={"source_model": source_model, "source_revision": source_revision,
                                              "precision": "float16", "scope": "encoder+classification-only"})
    if encoder_config is not None:
        shutil.copyfile(encoder_config, out / "encoder-config.json")
    return path


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--source", type=Path, required=True, help="the upstream model.safetensors")
    p.add_argument("--output", type=Path, default=Path("Artifacts"))
    p.add_argument("--encoder-config", type=Path, default=None)
    a = p.parse_args(argv)
    try:
        print(prepare_weights(a.source, a.output, a.encoder_config))
    except (RuntimeError, OSError) as e:
        sys.stderr.write(f"error: {e}\n")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
