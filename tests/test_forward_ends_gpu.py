"""The forward's ends (patch embedding, time and text embeddings, head,
unpatchify; models.py:1357-1384, :1827-1875, :2234-2257) run on the GPU
against the CPU restatements of tests/test_forward_ends_host.py."""
import pytest

import test_forward_ends_host as ends

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("check", [ends.check_patch_embedding_is_the_conv3d,
                                   ends.check_sinusoidal_embedding_closed_form,
                                   ends.check_time_embedding_fp32_mlp,
                                   ends.check_text_embedding_pads_then_mlp,
                                   ends.check_head_fp32,
                                   ends.check_unpatchify_index_map],
                         ids=lambda f: f.__name__[len("check_"):])
def test_forward_end_on_gpu(check):
    print(f"[case] {check.__name__} on cuda", flush=True)
    check("cuda")
