"""MI355X paged-attention serving stack: the host-side mirror of the reference's `src` package.

Import paths, class and function names follow jacobzhang22/efficient-inference-system so code
written against `src.cache`, `src.kernels`, `src.model`, `src.inference` and `src.serving` runs
unchanged; the `"hip_paged"` attention backend routes the hot path through libpaged_hip.so.
"""
