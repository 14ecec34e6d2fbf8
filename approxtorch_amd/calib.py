"""Post-training calibration of the quantization parameters (approxtorch/calib.py).

calibrate_int8 / calibrate_uint8 run a float model over calibration data,
collect per-layer activation statistics with forward hooks and return the
model's state_dict extended with the quantization parameters that
nn.Conv2d_int8 / nn.Conv2d_uint8 load (so a calibrated checkpoint loads into
a converted model unchanged).  Layer selection, batch handling, errors and
the state_dict layout follow the reference (calib.py:7-127 int8,
130-335 uint8).

The activation statistics of CUDA fp32 inputs come from the library's
device reductions (atx_absmax / atx_minmax) and stay on the device until
the end (the reference's int8 path syncs the host on every batch and layer);
other inputs use torch's reductions.  max / min are exact in any order, so
the statistics -- and the parameters derived from them -- are the
reference's, bit for bit.
"""
import torch
import torch.nn as nn

from .backend import _lib as L
from .backend import ops
from .nn.Conv2d_uint8 import uint8_qparams


def _absmax(x):
    """0-dim fp32 max |x| (NaN propagates like torch's max)."""
    if x.is_cuda and x.dtype == torch.float32 and x.numel() > 0:
        xc = x.contiguous()
        out = torch.empty((), dtype=torch.float32, device=x.device)
        L.call("atx_absmax", L.ptr(xc), xc.numel(), L.ptr(ops._reduce_ws(x.device)), L.ptr(out),
               L.stream_of(xc))
        return out
    return x.abs().max().to(torch.float32)


def _minmax(x):
    """(min, max) of x as 0-dim fp32 tensors."""
    if x.is_cuda and x.dtype == torch.float32 and x.numel() > 0:
        xc = x.contiguous()
        mn = torch.empty((), dtype=torch.float32, device=x.device)
        mx = torch.empty((), dtype=torch.float32, device=x.device)
        L.call("atx_minmax", L.ptr(xc), xc.numel(), L.ptr(ops._reduce_ws(x.device)), L.ptr(mn),
               L.ptr(mx), L.stream_of(xc))
        return mn, mx
    return x.amin().to(torch.float32), x.amax().to(torch.float32)


def calibrate_int8(model, data_loader, num_pictures, save_path, weight_bits=8):
    """min-max (absmax) calibration for Conv2d_int8 (calib.py:7-127).

    Skips the first nn.Conv2d; activations: per-tensor absmax / 127 (1.0 when
    the absmax is 0); weights: per-output-channel absmax / (2^(b-1) - 1) (1.0
    for all-zero channels).  Returns the state_dict with `<layer>.scale_x` and
    `<layer>.scale_w` inserted after each calibrated layer's last entry, and
    saves it to save_path."""
    if not 3 <= weight_bits <= 8:
        raise ValueError(f"weight_bits must be between 3 and 8, got {weight_bits}")
    model.eval()
    device = next(model.parameters()).device

    target_layers = {}
    first_conv_skipped = False
    for name, module in model.named_modules():
        if isinstance(module, nn.Conv2d):
            if not first_conv_skipped:
                first_conv_skipped = True
                print(f"[Skip] first Conv2d: {name}")
                continue
            target_layers[name] = module

    # running absmax per layer, kept on the layer's device; NaN batches are
    # ignored as the reference's `if cur > record` comparison ignores them
    absmax_record = {name: None for name in target_layers}

    def make_hook(layer_name):
        def hook(module, inputs, output):
            cur = _absmax(inputs[0].detach())
            rec = absmax_record[layer_name]
            if rec is None:
                rec = torch.zeros((), dtype=torch.float32, device=cur.device)
            absmax_record[layer_name] = torch.where(cur > rec, cur, rec)
        return hook

    qmax_w = 2 ** (weight_bits - 1) - 1
    hooks = [m.register_forward_hook(make_hook(n)) for n, m in target_layers.items()]
    seen = 0
    with torch.no_grad():
        for batch in data_loader:
            imgs = batch[0] if isinstance(batch, (list, tuple)) else batch
            imgs = imgs.to(device)
            model(imgs)
            seen += imgs.size(0)
            if seen >= num_pictures:
                break
    for h in hooks:
        h.remove()

    scale_x_dict = {}
    for name, rec in absmax_record.items():
        absmax = 0.0 if rec is None else float(rec.item())
        # python-double division, then fp32, as the reference's torch.tensor(scale)
        scale = absmax / 127.0 if absmax > 0 else 1.0
        scale_x_dict[name] = torch.tensor(scale)
        print(f"[scale_x] {name}: absmax={absmax:.6f}, scale={scale:.8f}")

    scale_w_dict = {}
    for name, module in target_layers.items():
        w = module.weight.detach()
        absmax_per_oc = w.abs().amax(dim=tuple(range(1, w.dim())))
        scale_w = absmax_per_oc / qmax_w
        scale_w = torch.where(scale_w > 0, scale_w, torch.ones_like(scale_w))
        scale_w_dict[name] = scale_w
        print(f"[scale_w] {name}: shape={tuple(scale_w.shape)}, "
              f"max={scale_w.max().item():.8f}, min={scale_w.min().item():.8f}")

    orig_state = model.state_dict()
    last_key_of_layer = {}
    for k in orig_state.keys():
        layer_name = k.rsplit(".", 1)[0]
        if layer_name in target_layers:
            last_key_of_layer[layer_name] = k
    new_state_dict = {}
    for k, v in orig_state.items():
        new_state_dict[k] = v
        layer_name = k.rsplit(".", 1)[0]
        if layer_name in target_layers and k == last_key_of_layer[layer_name]:
            new_state_dict[f"{layer_name}.scale_x"] = scale_x_dict[layer_name]
            new_state_dict[f"{layer_name}.scale_w"] = scale_w_dict[layer_name]

    torch.save(new_state_dict, save_path)
    print(f"[Save] saved to {save_path}")
    return new_state_dict


def calibrate_uint8(model, data_loader, num_pictures, save_path=None, ignore_first_conv=True):
    """Asymmetric uint8 calibration for Conv2d_uint8 (calib.py:130-335).

    Activations: per-tensor min/max; weights: per-output-channel min/max;
    ranges widened to include 0; scale / zero point from uint8_qparams with
    the zero point kept as an integer-valued fp32.  Every calibrated layer
    gets x_min/x_max/w_min/w_max (the statistics buffers) and
    scale_x/zero_x/scale_w/zero_w.  The model's train/eval flags are
    restored; num_pictures (None = the whole loader) truncates the last
    batch."""
    if num_pictures is not None:
        if isinstance(num_pictures, bool) or not isinstance(num_pictures, int):
            raise TypeError("num_pictures must be a positive int or None")
        if num_pictures <= 0:
            raise ValueError("num_pictures must be positive")

    first_parameter = next(model.parameters(), None)
    first_buffer = next(model.buffers(), None)
    if first_parameter is not None:
        device = first_parameter.device
    elif first_buffer is not None:
        device = first_buffer.device
    else:
        device = torch.device("cpu")

    target_layers = {}
    first_conv_seen = False
    for name, module in model.named_modules():
        if not isinstance(module, nn.Conv2d):
            continue
        if ignore_first_conv and not first_conv_seen:
            first_conv_seen = True
            print(f"[Skip] first Conv2d: {name or '<root>'}")
            continue
        first_conv_seen = True
        target_layers[name] = module
    if not target_layers:
        raise ValueError(
            "no Conv2d layers selected for uint8 calibration; if the model "
            "contains only one Conv2d, pass ignore_first_conv=False")

    x_min_record = {name: torch.tensor(float("inf"), dtype=torch.float32,
                                       device=m.weight.device)
                    for name, m in target_layers.items()}
    x_max_record = {name: torch.tensor(float("-inf"), dtype=torch.float32,
                                       device=m.weight.device)
                    for name, m in target_layers.items()}

    def make_hook(layer_name):
        def hook(module, inputs, output):
            if not inputs or not isinstance(inputs[0], torch.Tensor):
                raise TypeError(f"input of Conv2d '{layer_name}' must be a torch.Tensor")
            mn, mx = _minmax(inputs[0].detach())
            if not (torch.isfinite(mn) and torch.isfinite(mx)):
                raise ValueError(f"non-finite activation observed at Conv2d '{layer_name}'")
            x_min_record[layer_name] = torch.minimum(x_min_record[layer_name], mn)
            x_max_record[layer_name] = torch.maximum(x_max_record[layer_name], mx)
        return hook

    hooks = [m.register_forward_hook(make_hook(n)) for n, m in target_layers.items()]
    training_states = {module: module.training for module in model.modules()}
    seen = 0
    model.eval()
    try:
        with torch.no_grad():
            for batch in data_loader:
                images = batch[0] if isinstance(batch, (list, tuple)) else batch
                if not isinstance(images, torch.Tensor):
                    raise TypeError("calibration batch must be a Tensor or a list/tuple "
                                    "whose first element is a Tensor")
                if images.dim() == 0:
                    raise ValueError("calibration input must have a batch dimension")
                if num_pictures is not None:
                    remaining = num_pictures - seen
                    if remaining <= 0:
                        break
                    images = images[:remaining]
                if images.shape[0] == 0:
                    continue
                images = images.to(device)
                model(images)
                seen += images.shape[0]
                if num_pictures is not None and seen >= num_pictures:
                    break
    finally:
        for h in hooks:
            h.remove()
        for module, training in training_states.items():
            module.training = training
    if seen == 0:
        raise ValueError("data_loader yielded no calibration samples")

    qparams = {}
    for name, module in target_layers.items():
        observed_min, observed_max = x_min_record[name], x_max_record[name]
        if not (torch.isfinite(observed_min) and torch.isfinite(observed_max)):
            raise RuntimeError(f"Conv2d '{name}' did not run during calibration")
        x_min = torch.minimum(observed_min, torch.zeros_like(observed_min))
        x_max = torch.maximum(observed_max, torch.zeros_like(observed_max))
        weight = module.weight.detach()
        if not torch.isfinite(weight).all():
            raise ValueError(f"non-finite weight observed at Conv2d '{name}'")
        reduce_dims = tuple(range(1, weight.dim()))
        w_min = weight.amin(dim=reduce_dims).to(dtype=torch.float32)
        w_max = weight.amax(dim=reduce_dims).to(dtype=torch.float32)
        w_min = torch.minimum(w_min, torch.zeros_like(w_min))
        w_max = torch.maximum(w_max, torch.zeros_like(w_max))
        scale_x, zero_x = uint8_qparams(x_min, x_max)
        scale_w, zero_w = uint8_qparams(w_min, w_max)
        qparams[name] = {
            "x_min": x_min.detach().clone(), "x_max": x_max.detach().clone(),
            "w_min": w_min.detach().clone(), "w_max": w_max.detach().clone(),
            "scale_x": scale_x.detach().clone(),
            "zero_x": zero_x.to(dtype=torch.float32).detach().clone(),
            "scale_w": scale_w.detach().clone(),
            "zero_w": zero_w.to(dtype=torch.float32).detach().clone(),
        }
        print(f"[uint8 qparams] {name}: x=[{x_min.item():.6g}, {x_max.item():.6g}], "
              f"scale_x={scale_x.item():.8g}, zero_x={zero_x.item()}, "
              f"weight_channels={weight.shape[0]}, "
              f"zero_w=[{zero_w.min().item()}, {zero_w.max().item()}]")

    new_state_dict = model.state_dict()
    for name, layer_qparams in qparams.items():
        for field, value in layer_qparams.items():
            new_state_dict[f"{name}.{field}" if name else field] = value
    if save_path is not None:
        torch.save(new_state_dict, save_path)
        print(f"[Save] uint8 calibration parameters saved to {save_path}")
    return new_state_dict
