"""fdr_group_sum (grouped value heads: dq / dk summed over each q / k head's group) against
the same sum formed by torch in fp32, group members added in ascending order, then rounded
to bf16 once: bit for bit, for group sizes 1-4 and a token count that is not a multiple of
anything the kernel tiles by."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("G", [1, 2, 3, 4])
def test_group_sum_matches_a_sequential_fp32_sum(G):
    from rewy_amd import ops
    B, T, HQ = 2, 100, 3
    print(f"\n[group_sum] G={G}", flush=True)
    x = torch.randn(B, T, HQ * G, 128, generator=torch.Generator().manual_seed(G)).bfloat16()
    ref = torch.zeros(B, T, HQ, 128)
    xv = x.view(B, T, HQ, G, 128).float()
    for j in range(G):
        ref = ref + xv[:, :, :, j]
    got = ops.group_sum(x.cuda(), HQ)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), ref.bfloat16())
