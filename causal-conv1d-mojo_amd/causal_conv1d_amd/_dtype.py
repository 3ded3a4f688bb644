"""dtype codes shared with the C ABI (``include/cc1d.h``, ``enum cc1d_dtype``).

Same numbering as the reference's ``_DTYPE_CODE``
(``src/causal_conv1d_mojo/_dtype.py:16-20``).
"""

from __future__ import annotations

import torch

_DTYPE_CODE = {
    torch.float16: 0,
    torch.bfloat16: 1,
    torch.float32: 2,
}
