"""GLiNER-Decide encoder path on MI355X (gfx950): Python mirror of the
reference's Swift API over the HIP C-ABI (include/gliner_decide.h).

    from gliner_decide import GLiNERDecideClassifier, DecisionInput
    model = GLiNERDecideClassifier("decide-classification-fp16.safetensors")
    result = model.classify(DecisionInput(ids, mask, markers, marker_mask))

Importing this package needs no GPU; constructing the classifier or calling
a kernel needs the built library and a ROCm device, and raises otherwise.
"""

from ._native import EXPORTED_SYMBOLS, GlinerDecideError, lib, library_path  # noqa: F401
from .config import DeBERTaV2Configuration  # noqa: F401
from .decode import DecisionTask, Prediction, decode, make_batch_chunk, select_bucket  # noqa: F401


def __getattr__(name):
    # torch-dependent classes load lazily so `import gliner_decide` stays light.
    if name in ("GLiNERDecideClassifier", "DecisionInput", "InferenceResult", "ProfileEvent"):
        from . import classifier
        return getattr(classifier, name)
    if name == "FusedKernels":
        from .fused_kernels import FusedKernels
        return FusedKernels
    if name == "WeightStore":
        from .weights import WeightStore
        return WeightStore
    raise AttributeError(name)
