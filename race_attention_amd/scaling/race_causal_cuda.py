"""Drop-in for the reference module scaling/race_causal_cuda.py: callers that put this
directory on sys.path (e.g. RACE_SCALING_DIR, chat/nanochat/gpt.py:30-34) get the
MI355X implementation under the reference's import name."""
import os as _os
import sys as _sys

_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
if _ROOT not in _sys.path:
    _sys.path.insert(0, _ROOT)

from race_attention_amd.race_causal_cuda import (RaceCausalCuda, RaceCausalFn, _ext, fwd_chunk,  # noqa: E402,F401
                                                 race_backward, race_cuda_fused, race_fused_fwd)
