"""Post-training calibration of the quantization parameters (the API of
approxtorch/calib.py: calibrate_int8 at calib.py:7-127, calibrate_uint8 at
130-335).

A float model is run over calibration data while forward hooks feed every
selected conv layer's input to an observer of its range; the parameters that
nn.Conv2d_int8 / nn.Conv2d_uint8 load are derived from the observed ranges
and the weights and added to the model's state_dict, so a calibrated
checkpoint loads into a converted model unchanged.

The observers keep their running statistics on the layer's device: CUDA fp32
inputs are reduced by the library's kernels (atx_absmax / atx_minmax), other
inputs by torch, and nothing is read back until the parameters are formed.
max / min are exact in any order, so the statistics -- and the parameters --
are the reference's, bit for bit.
"""
import torch
import torch.nn as nn

from .backend import _lib as L
from .backend import ops
from .nn.Conv2d_uint8 import uint8_qparams


# ----------------------------------------------------------------- observers
def _device_reduce(x, want_minmax):
    """Reductions of a CUDA fp32 tensor by the library's kernels."""
    xc = x.contiguous()
    ws = ops._reduce_ws(x.device)
    if want_minmax:
        mn = torch.empty((), dtype=torch.float32, device=x.device)
        mx = torch.empty((), dtype=torch.float32, device=x.device)
        L.call("atx_minmax", L.ptr(xc), xc.numel(), L.ptr(ws), L.ptr(mn), L.ptr(mx),
               L.stream_of(xc))
        return mn, mx
    out = torch.empty((), dtype=torch.float32, device=x.device)
    L.call("atx_absmax", L.ptr(xc), xc.numel(), L.ptr(ws), L.ptr(out), L.stream_of(xc))
    return out


def _on_device(x):
    return x.is_cuda and x.dtype == torch.float32 and x.numel() > 0


class _AbsMaxObserver:
    """Largest |x| seen (0 before any input; a NaN statistic never replaces
    the record, as in the reference's `cur > record` comparison)."""

    def __init__(self, device):
        self.value = torch.zeros((), dtype=torch.float32, device=device)

    def update(self, x):
        cur = _device_reduce(x, False) if _on_device(x) else x.abs().max().to(torch.float32)
        cur = cur.to(self.value.device)
        self.value = torch.where(cur > self.value, cur, self.value)

    def absmax(self):
        return float(self.value.item())


class _MinMaxObserver:
    """Smallest / largest x seen; non-finite statistics are an error."""

    def __init__(self, device, layer_name):
        self.lo = torch.full((), float("inf"), dtype=torch.float32, device=device)
        self.hi = torch.full((), float("-inf"), dtype=torch.float32, device=device)
        self.layer_name = layer_name

    def update(self, x):
        if _on_device(x):
            mn, mx = _device_reduce(x, True)
        else:
            mn, mx = x.amin().to(torch.float32), x.amax().to(torch.float32)
        if not bool(torch.isfinite(mn) & torch.isfinite(mx)):
            raise ValueError(f"non-finite activation observed at Conv2d '{self.layer_name}'")
        self.lo = torch.minimum(self.lo, mn.to(self.lo.device))
        self.hi = torch.maximum(self.hi, mx.to(self.hi.device))

    def seen(self):
        return bool(torch.isfinite(self.lo) & torch.isfinite(self.hi))


# ------------------------------------------------------------- the pass
def _conv_layers(model, skip_first):
    """Conv2d layers in module order, optionally without the first one."""
    chosen = {}
    pending_skip = skip_first
    for name, module in model.named_modules():
        if not isinstance(module, nn.Conv2d):
            continue
        if pending_skip:
            pending_skip = False
            print(f"[Skip] first Conv2d: {name or '<root>'}")
            continue
        chosen[name] = module
    return chosen


def _batch_images(batch, checked):
    images = batch[0] if isinstance(batch, (list, tuple)) else batch
    if checked:
        if not isinstance(images, torch.Tensor):
            raise TypeError("calibration batch must be a Tensor or a list/tuple "
                            "whose first element is a Tensor")
        if images.dim() == 0:
            raise ValueError("calibration input must have a batch dimension")
    return images


def _calibration_pass(model, data_loader, device, observers, limit, exact_count, checked):
    """Runs the model (no grad) over data_loader with every observer fed its
    layer's input; stops once `limit` samples have run (None: the whole
    loader).  exact_count trims the last batch to the limit and skips empty
    batches.  Returns the number of samples that ran."""

    def feeder(name, obs):
        def hook(module, inputs, output):
            if checked and (not inputs or not isinstance(inputs[0], torch.Tensor)):
                raise TypeError(f"input of Conv2d '{name}' must be a torch.Tensor")
            obs.update(inputs[0].detach())
        return hook

    handles = [layer.register_forward_hook(feeder(name, obs))
               for name, (layer, obs) in observers.items()]
    seen = 0
    try:
        with torch.no_grad():
            for batch in data_loader:
                images = _batch_images(batch, checked)
                if exact_count and limit is not None:
                    if limit - seen <= 0:
                        break
                    images = images[:limit - seen]
                if exact_count and images.shape[0] == 0:
                    continue
                images = images.to(device)
                model(images)
                seen += images.size(0)
                if limit is not None and seen >= limit:
                    break
    finally:
        for h in handles:
            h.remove()
    return seen


def _with_entries(state, entries, after_layer):
    """state_dict plus entries {layer: {field: tensor}}; after_layer places a
    layer's fields right after its last existing entry (the int8 layout),
    otherwise they are added (or overwritten) at the end."""
    if not after_layer:
        for layer, fields in entries.items():
            for field, value in fields.items():
                state[f"{layer}.{field}" if layer else field] = value
        return state
    owner = {key: key.rsplit(".", 1)[0] for key in state}
    last = {}
    for key, layer in owner.items():
        if layer in entries:
            last[layer] = key
    out = {}
    for key, value in state.items():
        out[key] = value
        layer = owner[key]
        if last.get(layer) == key:
            for field, extra in entries[layer].items():
                out[f"{layer}.{field}"] = extra
    return out


def _channel_absmax_scale(weight, qmax):
    """Per-output-channel absmax / qmax, 1.0 for an all-zero channel."""
    s = weight.abs().amax(dim=tuple(range(1, weight.dim()))) / qmax
    return torch.where(s > 0, s, torch.ones_like(s))


# ------------------------------------------------------------------ int8
def calibrate_int8(model, data_loader, num_pictures, save_path, weight_bits=8):
    """min-max (absmax) calibration for Conv2d_int8.

    The first nn.Conv2d is skipped; activations get a per-tensor scale
    absmax / 127 (1.0 when the absmax is 0), weights a per-output-channel
    absmax / (2^(b-1) - 1) (1.0 for all-zero channels).  Whole batches run
    until num_pictures samples have been seen.  Returns the state_dict with
    `<layer>.scale_x` and `<layer>.scale_w` placed after each calibrated
    layer's entries, and saves it to save_path."""
    if not 3 <= weight_bits <= 8:
        raise ValueError(f"weight_bits must be between 3 and 8, got {weight_bits}")
    model.eval()
    device = next(model.parameters()).device
    layers = _conv_layers(model, skip_first=True)
    observers = {name: (layer, _AbsMaxObserver(layer.weight.device))
                 for name, layer in layers.items()}
    _calibration_pass(model, data_loader, device, observers, num_pictures, exact_count=False,
                      checked=False)

    qmax_w = 2 ** (weight_bits - 1) - 1
    entries = {}
    for name, (layer, obs) in observers.items():
        absmax = obs.absmax()
        # the reference divides in python doubles and stores torch.tensor(scale)
        scale = absmax / 127.0 if absmax > 0 else 1.0
        scale_w = _channel_absmax_scale(layer.weight.detach(), qmax_w)
        entries[name] = {"scale_x": torch.tensor(scale), "scale_w": scale_w}
        print(f"[scale_x] {name}: absmax={absmax:.6f}, scale={scale:.8f}")
        print(f"[scale_w] {name}: shape={tuple(scale_w.shape)}, "
              f"max={scale_w.max().item():.8f}, min={scale_w.min().item():.8f}")

    state = _with_entries(model.state_dict(), entries, after_layer=True)
    torch.save(state, save_path)
    print(f"[Save] saved to {save_path}")
    return state


# ----------------------------------------------------------------- uint8
def _model_device(model):
    for t in model.parameters():
        return t.device
    for t in model.buffers():
        return t.device
    return torch.device("cpu")


def _uint8_layer_qparams(name, layer, obs):
    """Effective ranges (including 0) and qparams of one layer."""
    if not obs.seen():
        raise RuntimeError(f"Conv2d '{name}' did not run during calibration")
    zero = torch.zeros((), dtype=torch.float32, device=obs.lo.device)
    x_lo, x_hi = torch.minimum(obs.lo, zero), torch.maximum(obs.hi, zero)
    weight = layer.weight.detach()
    if not torch.isfinite(weight).all():
        raise ValueError(f"non-finite weight observed at Conv2d '{name}'")
    dims = tuple(range(1, weight.dim()))
    w_lo = weight.amin(dim=dims).to(torch.float32).clamp(max=0.0)
    w_hi = weight.amax(dim=dims).to(torch.float32).clamp(min=0.0)
    sx, zx = uint8_qparams(x_lo, x_hi)
    sw, zw = uint8_qparams(w_lo, w_hi)
    fields = {"x_min": x_lo, "x_max": x_hi, "w_min": w_lo, "w_max": w_hi,
              "scale_x": sx, "zero_x": zx.to(torch.float32), "scale_w": sw,
              "zero_w": zw.to(torch.float32)}
    print(f"[uint8 qparams] {name}: x=[{x_lo.item():.6g}, {x_hi.item():.6g}], "
          f"scale_x={sx.item():.8g}, zero_x={fields['zero_x'].item()}, "
          f"weight_channels={weight.shape[0]}, "
          f"zero_w=[{fields['zero_w'].min().item()}, {fields['zero_w'].max().item()}]")
    return {k: v.detach().clone() for k, v in fields.items()}


def calibrate_uint8(model, data_loader, num_pictures, save_path=None, ignore_first_conv=True):
    """Asymmetric uint8 calibration for Conv2d_uint8.

    Activations: per-tensor min/max; weights: per-output-channel min/max;
    ranges widened to include 0; scale / zero point from uint8_qparams, the
    zero point an integer-valued fp32.  Every calibrated layer gets
    x_min/x_max/w_min/w_max (the statistics buffers) and
    scale_x/zero_x/scale_w/zero_w.  num_pictures (None = the whole loader)
    trims the last batch; every module's train/eval flag is restored."""
    if num_pictures is not None:
        if isinstance(num_pictures, bool) or not isinstance(num_pictures, int):
            raise TypeError("num_pictures must be a positive int or None")
        if num_pictures <= 0:
            raise ValueError("num_pictures must be positive")
    device = _model_device(model)
    layers = _conv_layers(model, skip_first=ignore_first_conv)
    if not layers:
        raise ValueError(
            "no Conv2d layers selected for uint8 calibration; if the model "
            "contains only one Conv2d, pass ignore_first_conv=False")
    observers = {name: (layer, _MinMaxObserver(layer.weight.device, name))
                 for name, layer in layers.items()}

    flags = [(m, m.training) for m in model.modules()]
    model.eval()
    try:
        seen = _calibration_pass(model, data_loader, device, observers, num_pictures,
                                 exact_count=True, checked=True)
    finally:
        for m, was_training in flags:
            m.training = was_training
    if seen == 0:
        raise ValueError("data_loader yielded no calibration samples")

    entries = {name: _uint8_layer_qparams(name, layer, obs)
               for name, (layer, obs) in observers.items()}
    state = _with_entries(model.state_dict(), entries, after_layer=False)
    if save_path is not None:
        torch.save(state, save_path)
        print(f"[Save] uint8 calibration parameters saved to {save_path}")
    return state
