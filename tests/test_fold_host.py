"""Host-side choice of the folded KV write (no GPU needed).

``forward_mixed`` and ``Attention.forward`` fold the store into the attention
launch only for new K/V rows stored back to back (``slo_attn.ops.foldable``);
views of a fused projection output keep the separate store launch.
"""
import torch

from slo_attn.ops import foldable


def test_contiguous_rows_fold():
    k = torch.zeros(5, 8, 128, dtype=torch.bfloat16)
    assert foldable(k, k.clone())


def test_strided_views_and_other_dtypes_do_not_fold():
    qkv = torch.zeros(5, 48, 128, dtype=torch.bfloat16)  # q, k, v heads of a fused projection
    k, v = qkv[:, 32:40], qkv[:, 40:48]
    assert not foldable(k, v)
    kf = torch.zeros(5, 8, 128, dtype=torch.float32)
    assert not foldable(kf, kf.clone())
    kt = torch.zeros(5, 128, 8, dtype=torch.bfloat16).transpose(1, 2)  # heads not contiguous
    assert not foldable(kt, kt)
