"""skyla_hip: host side of the MI355X (gfx950) backend for Skyla's quantized weight path.

abi     -- ctypes binding of include/skyla_hip.h (the backend surface: Context, Buffer,
           Pipeline, Recorder, Recording)
engine  -- the skyla-engine side of the path: planner layout, pipelines and tactics,
           the push words and grids of every weight-path dispatch, the arena layout
synth   -- seeded synthetic GGUF blocks and activations for the benchmark configs
"""
from .abi import Buffer, Context, Pipeline, Recorder, Recording, SkylaHipError, load_library  # noqa: F401
from .engine import DType  # noqa: F401
