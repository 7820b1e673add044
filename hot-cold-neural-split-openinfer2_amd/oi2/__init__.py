"""MI355X (gfx950) hot/cold sparse-FFN decode path behind OpenInfer2's
interfaces: ColdWeightStore (splitter.py), SparseFFNLayer / sparse_ffn
(engine.py), PredictorRegistry / NeuronPredictor (predictor.py) and the
decode attention GroupedQueryAttention (engine.py), composed per layer
by DecoderStep."""
from . import format
from ._lib import OI2Error, load_library
from .attention import GroupedQueryAttention, rope_tables
from .decode_step import DecoderStep
from .format import (ALIGN_BYTES, HIDDEN_DIM, NEURON_RECORD_BYTES, PAGE_ALIGN, quantize_int4)
from .hot import HotWeights
from .layer import ColdNeurons, SparseFFNLayer, sparse_ffn
from .predictor import NeuronPredictor, PredictorRegistry
from .stack import DecodeStack, StackLayer
from .store import ColdSection, ColdWeightStore

__all__ = [
    "format", "OI2Error", "load_library", "ALIGN_BYTES", "HIDDEN_DIM", "NEURON_RECORD_BYTES",
    "PAGE_ALIGN", "quantize_int4", "HotWeights", "ColdNeurons", "SparseFFNLayer", "sparse_ffn",
    "NeuronPredictor", "PredictorRegistry", "DecodeStack", "StackLayer", "ColdSection",
    "ColdWeightStore", "GroupedQueryAttention", "rope_tables", "DecoderStep",
]
