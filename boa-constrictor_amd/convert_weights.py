"""Convert a BoaConstrictor mambav1 PyTorch checkpoint to the BOA weight file.

Same command line and output as the reference converter
(portability_solved_cpp/convert_boa_weights.py:153-257) for the mambav1
backbone:

    python convert_weights.py --model model.pt --output model.bin [--fp16]

* header "BOA\\x00" (fp32) or "BOA\\x01" (fp16); fp16 is chosen when the
  checkpoint's first weight tensor is fp16 or when --fp16 is given
  (convert_boa_weights.py:174-179);
* tensors in the order embedding, per block (ln1, in_proj w/b, conv1d w/b,
  x_proj, dt_proj w/b, A_log, D, out_proj w/b, ln2, ff.0 w/b, ff.2 w/b),
  head.0 w/b, head.2 w/b; a missing in_proj / out_proj bias is written as
  zeros (convert_boa_weights.py:37-88, 186-239);
* "model_state_dict" / "state_dict" wrappers are unwrapped (:157-160).

Unlike the reference the checkpoint is read with torch.load(weights_only=True),
which executes nothing from the file; other backbones (LSTM, GRU, minGRU) are
rejected because the HIP path runs mambav1 only.  The written size is checked
against the dimensions read from the checkpoint.
"""
import argparse
import os
import sys

import numpy as np

import synth


def load_state_dict(path: str):
    import torch
    sd = torch.load(path, map_location="cpu", weights_only=True)
    if isinstance(sd, dict) and "model_state_dict" in sd:
        sd = sd["model_state_dict"]
    elif isinstance(sd, dict) and "state_dict" in sd:
        sd = sd["state_dict"]
    if not isinstance(sd, dict):
        raise ValueError(f"{path}: not a state dict")
    return sd


def detect_backbone(sd) -> str:
    """Key-based detection as convert_boa_weights.py:23-34."""
    for k in sd:
        if ".mamba." in k:
            return "mamba"
        if ".lstm." in k:
            return "lstm"
        if ".gru." in k and ".mingru." not in k:
            return "gru"
        if ".mingru." in k:
            return "mingru"
    return "mamba"


def model_dims(sd):
    """(d_model, n_layers, d_state) of a mambav1 state dict."""
    d_model = int(sd["embedding.weight"].shape[1])
    n_layers = 0
    while f"blocks.{n_layers}.ln1.weight" in sd:
        n_layers += 1
    d_state = int(sd["blocks.0.mamba.A_log"].shape[1]) if n_layers else 16
    return d_model, n_layers, d_state


def checkpoint_is_fp16(sd) -> bool:
    import torch
    key = next(k for k in sd if "weight" in k)
    return sd[key].dtype == torch.float16


def convert(model_path: str, output_path: str, fp16: bool = False, backbone: str = None) -> dict:
    sd = load_state_dict(model_path)
    bb = backbone or detect_backbone(sd)
    if bb not in ("mamba", "mambav1"):
        raise ValueError(f"backbone {bb!r} is not supported (mambav1 only)")
    use_fp16 = fp16 or checkpoint_is_fp16(sd)
    d_model, n_layers, d_state = model_dims(sd)
    tensors, n = synth.convert_state_dict(sd, d_state)
    size = synth.write_weights(output_path, tensors, fp16=use_fp16)
    want = synth.expected_weight_bytes(d_model, n_layers, d_state, fp16=use_fp16)
    if size != want:
        os.remove(output_path)
        raise ValueError(f"wrote {size} bytes, the d_model={d_model} n_layers={n_layers} "
                         f"d_state={d_state} layout needs {want}")
    return dict(d_model=d_model, n_layers=n_layers, d_state=d_state,
                precision="fp16" if use_fp16 else "fp32", bytes=size)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Convert BoaConstrictor PyTorch weights to the "
                                             "BOA binary weight file")
    ap.add_argument("--model", required=True, help="path to the .pt checkpoint")
    ap.add_argument("--output", required=True, help="path of the .bin to write")
    ap.add_argument("--fp16", action="store_true",
                    help="write fp16 (auto-detected from the checkpoint if not set)")
    ap.add_argument("--backbone", default=None, help="mamba (default: detected from the keys)")
    args = ap.parse_args(argv)
    try:
        info = convert(args.model, args.output, args.fp16, args.backbone)
    except (ValueError, KeyError, OSError) as e:
        print(f"ERROR: {e}", file=sys.stderr)
        return 1
    print(f"Saved {args.output}: d_model={info['d_model']} n_layers={info['n_layers']} "
          f"d_state={info['d_state']} {info['precision']} ({info['bytes']} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
