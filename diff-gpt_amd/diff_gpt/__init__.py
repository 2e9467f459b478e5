"""diff-gpt's inference API on MI355X (gfx950).

Drop-in for the ``diff_gpt`` package of fxeqxmulfx/diff-gpt on its attention
hot path: the module paths, class names, signatures, parameter names and
assertion messages of ``diff_gpt.model.*`` and ``diff_gpt.sampler.*`` are kept,
while RoPE, QK-norm, the KV-cache append and all attention run in the HIP
library ``libdgattn.so`` (see ``diff_gpt._native``).
"""
