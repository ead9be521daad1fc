"""Import name of the package kept in the directory `qwen-warp_amd/` (a hyphen cannot appear in a Python
import name): `import qwen_warp_amd` resolves its submodules from that directory."""
import os as _os

__path__ = [_os.path.join(_os.path.dirname(_os.path.abspath(__file__)), "qwen-warp_amd")]

from qwen_warp_amd.sampling import (TF_BROKEN, TF_RESCAN, TF_SPLIT_SELECT, TF_STAGED_DRAW, GenParams, PackedBatch, ProcState, RowSpec, Sampler, SeqSampler,  # noqa: E402,F401
                                    ValidationError, check_supported, draft_row, make_procs, make_sampling, row_from_params)
from qwen_warp_amd.pld import DevicePld  # noqa: E402,F401
from qwen_warp_amd.finish import StepBook  # noqa: E402,F401
from qwen_warp_amd.head import HeadSelect  # noqa: E402,F401
