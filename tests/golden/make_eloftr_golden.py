# SPDX-License-Identifier: Unlicense
"""Write tests/golden/eloftr_golden.npz: float64 outputs of Hugging Face
transformers' EfficientLoFTR (the implementation whose tensor names and
layers the reference's eloftr.c follows, eloftr.c:10-23 of
i.coregistration.opencl) with the seeded random-init weights of synth.py,
on the seeded synthetic pair at a small non-square tile:

* backbone: 1/8 features of both images (stage-3 output);
* coarse: both images after the 4 self + cross aggregated-attention layers;
* fine: the FPN fusion output (64 x H x W), sampled at fixed positions.

Built from the library's default config, no download. Coarse pairing and
fine matching are not taken from transformers (the reference follows the
authors' code there, eloftr.c:19-23). The weights and images are not
stored: they are regenerated from their seeds; their checksums are, so a
change of generator is caught.

    python tests/golden/make_eloftr_golden.py
"""

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / "i.coregistration.opencl_amd"))

import synth  # noqa: E402

H, W = 64, 96
NSAMPLE = 4096
SAMPLE_SEED = 7


def checksum(d):
    return np.array([float(np.sum(np.asarray(v, np.float64) ** 2)) for _, v in sorted(d.items())])


def main():
    import torch
    from transformers.models.efficientloftr import configuration_efficientloftr as c
    from transformers.models.efficientloftr import modeling_efficientloftr as m

    w = synth.eloftr_weights_calibrated()
    g0, g1, _ = synth.eloftr_pair(H, W)
    model = m.EfficientLoFTRForKeypointMatching(c.EfficientLoFTRConfig()).double().eval()
    missing, unexpected = model.load_state_dict(
        {k: torch.from_numpy(v.astype(np.float64)) for k, v in w.items()}, strict=False)
    assert not unexpected and all(k.endswith("num_batches_tracked") for k in missing)
    px = torch.from_numpy(np.stack([g0, g1]).astype(np.float64))[None, :, None]
    with torch.no_grad():
        bb = model.efficientloftr.backbone(px.reshape(2, 1, H, W))[-1]
        out = model.efficientloftr(px)
        coarse = out.feature_maps[0][0]
        res = list(reversed(out.feature_maps[1:]))
        fine = model.refinement_layer.forward_pyramid(
            out.feature_maps[0].reshape(2, 256, H // 8, W // 8) / 16.0, res)
    rng = np.random.default_rng(SAMPLE_SEED)
    idx = rng.choice(64 * H * W, NSAMPLE, replace=False)
    np.savez_compressed(
        HERE / "eloftr_golden.npz",
        H=H, W=W,
        weights_checksum=checksum(w),
        images_checksum=checksum({"0": g0, "1": g1}),
        backbone=bb.numpy().astype(np.float32),
        coarse=coarse.numpy().astype(np.float32),
        fine_idx=idx.astype(np.int64),
        fine=fine.reshape(2, -1).numpy()[:, idx].astype(np.float32),
    )
    print(f"written {HERE / 'eloftr_golden.npz'}")


if __name__ == "__main__":
    main()
