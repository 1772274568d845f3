"""TensorFlow module of the MI355X Sdpa / SdpaGrad ops.

The reference's Python interface, unchanged (README.md:28-56, test.py:12-30):
``sdpa(q, k, v, seed, offset, dropout=, scale=, causal_mask=)`` returns
``(o, stats)``, and the gradient registered for ``Sdpa`` calls ``SdpaGrad``
with the forward op's inputs, outputs and attributes and returns
``dq, dk, dv, None, None`` (no gradient for seed and offset).  Only the
library path differs: ``sdpa_rocm.so``, built by ``build.sh`` next to this
file.
"""
from __future__ import annotations

import os

import tensorflow as tf

LIB_PATH = os.environ.get("SDPA_ROCM_LIB",
                          os.path.join(os.path.dirname(os.path.abspath(__file__)), "sdpa_rocm.so"))
mod = tf.load_op_library(LIB_PATH)


def sdpa(q: tf.Tensor, k: tf.Tensor, v: tf.Tensor, seed: tf.Tensor, offset: tf.Tensor,
         dropout: float = 0.0, scale: float = 1.0, causal_mask: bool = False):
    """o [B, S_q, D_v] and stats [B, S_q] of softmax(scale q k^T) v with the
    op's dropout (keyed on seed + offset) and top-left causal mask."""
    return mod.sdpa(q, k, v, seed, offset, dropout=dropout, scale=scale, causal_mask=causal_mask)


@tf.RegisterGradient("Sdpa")
def _sdpa_grad(op: tf.Operation, d_o, *unused_d_stats):
    q, k, v, seed, offset = op.inputs
    o, stats = op.outputs
    dq, dk, dv = mod.sdpa_grad(q, k, v, o, stats, d_o, seed, offset,
                               dropout=op.get_attr("dropout"), scale=op.get_attr("scale"),
                               causal_mask=op.get_attr("causal_mask"))
    return dq, dk, dv, None, None
