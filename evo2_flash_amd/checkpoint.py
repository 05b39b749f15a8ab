"""Converted Evo 2 checkpoints, as the Hyena mixers consume them.

A converted checkpoint is a directory (convert.py:396-678 writes it):

  config.json                                  StripedHyena2Config fields, including
                                               the fp8 marker `hyena_in_proj_fp8`
  model.safetensors                            every weight under its model name
  metadata/hyena_in_proj_fp8_meta.safetensors  Transformer Engine scale audit of an
                                               fp8 checkpoint (never a weight shard)

The keys of one Hyena layer i (convert.py:465-494, 175-209), under
`model.layers.{i}.mixer.`:

  in_proj.weight         (3H, H) float8_e4m3fn (fp8 checkpoints) or bf16
  in_proj.weight_scale   (1,) fp32 dequantisation scale = TE scale_inv_fwd[1]
  in_proj.input_scale    (1,) fp32 dequantisation scale = TE scale_inv_fwd[0]
  in_proj_token_table    (vocab, 3H) bf16, layer 0 of FP8-surgery checkpoints only,
                         in place of in_proj (config.py:73-80, convert.py:712-780)
  in_proj_emul_weight_t  (H, 3H) bf16 E4M3 values, K-major, in place of in_proj for
                         `hyena_fp8_emulated_layers`; (H, n) beside a bf16 in_proj for
                         `hyena_fp8_emulated_channels` {i: n} (mixers.py:768-800)
  in_proj_emul_scales    (2,) fp32 [input_scale, weight_scale] of the emulated GEMM
  in_proj_emul_cols      (n,) int64 output channels the emulated GEMM overwrites
  short_filter.weight    (3H, 1, 3) bf16
  conv.weight            (H, 1, K) bf16, hcs / hcm, cross-correlation order
  D                      (H,) bf16, hcm and hcl
  log_poles              (H, S, 1) fp32, hcl
  residues               (H, S) fp32, hcl
  out_proj.weight        (H, H) bf16, out_proj.bias (H,) bf16

`short_filter.weight` and `conv.weight` load into the bare parameters
`short_filter` and `conv` (model.py:366-370).  Tensors are read with
safetensors, which executes nothing from the file; only the requested layer's
tensors are materialised.
"""

import json
import os

import torch

from .config import FP8_META_FILENAME, HyenaConfig

E4M3 = torch.float8_e4m3fn
CONFIG_FILE = "config.json"
WEIGHTS_FILE = "model.safetensors"
TOKEN_TABLE = "in_proj_token_table"


def read_config(path):
    """HyenaConfig of a converted checkpoint directory (or a config.json path),
    validated as the reference validates it (config.py:95-170)."""
    f = path if path.endswith(".json") else os.path.join(path, CONFIG_FILE)
    with open(f) as fh:
        return HyenaConfig.from_dict(json.load(fh))


def mixer_prefix(i):
    return f"model.layers.{i}.mixer."


def param_name(key, prefix):
    """Checkpoint key -> mixer parameter name (model.py:366-370)."""
    name = key[len(prefix):]
    if name in ("short_filter.weight", "conv.weight"):
        name = name[: -len(".weight")]
    return name


def expected_params(cfg, i):
    """{mixer parameter name: (shape, dtype)} a converted checkpoint holds
    for Hyena layer i under cfg (convert.py:465-494, 175-209)."""
    kind = cfg.layer_kind(i)
    if kind == "attn":
        raise ValueError(f"layer {i} is an attention layer")
    H, S = cfg.hidden_size, cfg.state_size
    bf16, f32 = torch.bfloat16, torch.float32
    p = {}
    n_emul = cfg.hyena_fp8_emulated_channels.get(i, 0)
    if i in cfg.hyena_token_table_layers:
        p[TOKEN_TABLE] = ((cfg.vocab_size, 3 * H), bf16)
    elif i in cfg.hyena_fp8_emulated_layers:
        p["in_proj_emul_weight_t"] = ((H, 3 * H), bf16)
        p["in_proj_emul_scales"] = ((2,), f32)
    elif n_emul:
        p["in_proj.weight"] = ((3 * H, H), bf16)
        p["in_proj_emul_weight_t"] = ((H, n_emul), bf16)
        p["in_proj_emul_scales"] = ((2,), f32)
        p["in_proj_emul_cols"] = ((n_emul,), torch.int64)
    elif cfg.use_fp8_input_projections:
        p["in_proj.weight"] = ((3 * H, H), E4M3)
        p["in_proj.weight_scale"] = ((1,), f32)
        p["in_proj.input_scale"] = ((1,), f32)
    else:
        p["in_proj.weight"] = ((3 * H, H), bf16)
    p["short_filter"] = ((3 * H, 1, cfg.short_filter_length), bf16)
    if kind == "hcl":
        p["log_poles"] = ((H, S, 1), f32)
        p["residues"] = ((H, S), f32)
    else:
        p["conv"] = ((H, 1, cfg.inner_filter_length(i)), bf16)
    if kind in ("hcm", "hcl"):
        p["D"] = ((H,), bf16)
    p["out_proj.weight"] = ((H, H), bf16)
    p["out_proj.bias"] = ((H,), bf16)
    return p


def _safe_open(path):
    from safetensors import safe_open

    return safe_open(path, framework="pt", device="cpu")


def load_mixer_params(path, i, cfg=None, device="cpu"):
    """{mixer parameter name: tensor} of Hyena layer i from a converted
    checkpoint directory, checked against the layout the converter writes:
    a missing, unexpected, mis-shaped or mis-typed tensor raises ValueError,
    as does a non-positive or non-finite fp8 scale."""
    cfg = cfg or read_config(path)
    want = expected_params(cfg, i)
    prefix = mixer_prefix(i)
    out = {}
    with _safe_open(os.path.join(path, WEIGHTS_FILE)) as f:
        keys = [k for k in f.keys() if k.startswith(prefix)]
        for k in keys:
            name = param_name(k, prefix)
            if name not in want:
                raise ValueError(f"unexpected checkpoint key {k!r} for a "
                                 f"{cfg.layer_kind(i)} layer")
            t = f.get_tensor(k)
            shape, dtype = want[name]
            if tuple(t.shape) != shape or t.dtype != dtype:
                raise ValueError(f"{k}: expected {shape} {dtype}, got {tuple(t.shape)} {t.dtype}")
            out[name] = t
    missing = sorted(set(want) - set(out))
    if missing:
        raise ValueError(f"layer {i}: checkpoint is missing {[prefix + m for m in missing]}")
    for name in ("in_proj.weight_scale", "in_proj.input_scale"):
        if name in out and not (torch.isfinite(out[name]).all() and (out[name] > 0).all()):
            raise ValueError(f"{prefix}{name} must be positive and finite, got {out[name]}")
    return {k: v.to(device) for k, v in out.items()}


def load_fp8_audit(path, cfg=None, tol=0.0):
    """The Transformer Engine scale audit of an fp8 checkpoint
    (metadata/hyena_in_proj_fp8_meta.safetensors, convert.py:198-207, 645-651),
    as {layer: {"scale_fwd", "scale_inv_fwd", "amax_history_fwd"}}, checked
    against the converter's contract: every Hyena layer present, shapes (3,),
    (3,), (16, 3), scale_fwd * scale_inv_fwd = 1 within 2e-3
    (convert.py:134-143), and the checkpoint's input_scale / weight_scale
    equal to scale_inv_fwd[0] / [1] (to `tol`, 0 = bit-exact)."""
    cfg = cfg or read_config(path)
    if not cfg.use_fp8_input_projections:
        raise ValueError("not an fp8 checkpoint: no hyena_in_proj_fp8 metadata")
    hyena = cfg.hyena_layers()
    audit = {}
    with _safe_open(os.path.join(path, FP8_META_FILENAME)) as f:
        keys = set(f.keys())
        want = {f"layers.{i}.{n}" for i in hyena
                for n in ("scale_fwd", "scale_inv_fwd", "amax_history_fwd")}
        if keys != want:
            raise ValueError(f"fp8 audit layers do not match the layer map: missing "
                             f"{sorted(want - keys)}, unexpected {sorted(keys - want)}")
        for i in hyena:
            rec = {n: f.get_tensor(f"layers.{i}.{n}").float()
                   for n in ("scale_fwd", "scale_inv_fwd", "amax_history_fwd")}
            for n, shape in (("scale_fwd", (3,)), ("scale_inv_fwd", (3,)),
                             ("amax_history_fwd", (16, 3))):
                if tuple(rec[n].shape) != shape:
                    raise ValueError(f"layers.{i}.{n} must have shape {shape}")
                if not torch.isfinite(rec[n]).all():
                    raise ValueError(f"layers.{i}.{n} contains non-finite values")
            if not torch.allclose(rec["scale_fwd"] * rec["scale_inv_fwd"], torch.ones(3),
                                  rtol=2e-3, atol=2e-3):
                raise ValueError(f"layers.{i}: scale_inv_fwd is not reciprocal to scale_fwd")
            audit[i] = rec
    with _safe_open(os.path.join(path, WEIGHTS_FILE)) as f:
        for i in hyena:
            p = mixer_prefix(i) + "in_proj."
            for name, j in (("input_scale", 0), ("weight_scale", 1)):
                got = f.get_tensor(p + name).float().reshape(())
                ref = audit[i]["scale_inv_fwd"][j]
                if (got - ref).abs() > tol * ref.abs():
                    raise ValueError(f"{p}{name} = {got.item()} but the audit's "
                                     f"scale_inv_fwd[{j}] = {ref.item()}")
    return audit


def load_hyena_mixers(path, device, cfg=None, quant_config=None, layers=None, name_prefix=""):
    """Build and load the Hyena mixers of a converted checkpoint:
    {layer index: HyenaFIRMixer | HyenaIIRMixer} with the checkpoint's
    weights on `device` (attention layers are not part of this path).  Layer i
    registers for the forward context as `{name_prefix}model.layers.{i}.mixer`,
    its module path in the model (mixers.py:806-810)."""
    from .mixers import load_mixer_params as _load, make_mixer

    cfg = cfg or read_config(path)
    out = {}
    for i in (layers if layers is not None else cfg.hyena_layers()):
        m = make_mixer(cfg, i, prefix=f"{name_prefix}model.layers.{i}.mixer",
                       quant_config=quant_config, device=device)
        out[i] = _load(m, load_mixer_params(path, i, cfg, device=device))
    return out
