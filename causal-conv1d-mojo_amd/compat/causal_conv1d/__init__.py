"""``import causal_conv1d`` namespace for code written against the upstream
Tri Dao ``causal-conv1d`` package, served by the gfx950 kernels of
``causal_conv1d_amd``.

Mirrors the reference's compatibility package
(``compat/src/causal_conv1d/__init__.py:24-48``): it re-exports the same five
names (not the varlen helpers) and refuses to load when the upstream
package's ``causal_conv1d_interface.py`` sits in the same directory, since two
installs sharing the ``causal_conv1d`` directory would mix modules of both.

Put ``causal-conv1d-mojo_amd/compat`` on ``sys.path`` (next to
``causal-conv1d-mojo_amd``) to use it.
"""

from __future__ import annotations

from pathlib import Path as _Path

if (_Path(__file__).resolve().parent / "causal_conv1d_interface.py").is_file():
    raise ImportError(
        "Both `causal-conv1d` (upstream Tri Dao) and the causal_conv1d_amd compatibility "
        "namespace are installed in the same `causal_conv1d` directory. Uninstall one of them."
    )

from causal_conv1d_amd import (  # noqa: E402
    __version__,
    causal_conv1d_fn,
    causal_conv1d_ref,
    causal_conv1d_update,
    causal_conv1d_update_ref,
)

__all__ = [
    "__version__",
    "causal_conv1d_fn",
    "causal_conv1d_ref",
    "causal_conv1d_update",
    "causal_conv1d_update_ref",
]
