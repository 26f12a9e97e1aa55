"""Argument checks shared by the three API functions.

Restates the reference's error conventions
(flywheel_tpu/softmax_attention/inputs.py:61-88, 218-251): NotImplementedError
for unsupported features, ValueError for malformed arguments.
"""

import math

import torch


def as_tensor(x):
    """Tensors pass through; DLPack-capable arrays are imported zero-copy."""
    if x is None or isinstance(x, torch.Tensor):
        return x
    if hasattr(x, "__dlpack__"):
        return torch.from_dlpack(x)
    return torch.as_tensor(x)


def check_common_kwargs(
    window_size,
    dropout_p=0.0,
    softcap=0.0,
    alibi_slopes=None,
    deterministic=False,
    return_attn_probs=False,
):
    """`inputs.py:218-251`: returns window_size as a tuple."""
    if dropout_p != 0.0:
        raise NotImplementedError("dropout_p is not supported.")
    window_size = tuple(window_size)
    if len(window_size) != 2 or any(b != -1 and b < 0 for b in window_size):
        raise ValueError(
            "window_size must be a 2-tuple of -1 (unbounded) or non-negative"
            f" ints; got {window_size}."
        )
    if softcap < 0.0:
        raise ValueError(f"softcap must be non-negative; got {softcap}.")
    if alibi_slopes is not None:
        raise NotImplementedError("alibi_slopes is not supported.")
    if deterministic:
        raise NotImplementedError(
            "deterministic is not supported; the forward kernels are deterministic already."
        )
    if return_attn_probs:
        raise NotImplementedError("return_attn_probs is not supported.")
    return tuple(int(b) for b in window_size)


def descale_scalar(descale, arg_name, device=None):
    """`inputs.py:61-72`: one per-tensor descale; None is 1.

    A Python number comes back as a float (passed to the kernels by value).
    A tensor or array stays a device value: it comes back as a (1,) float32
    tensor on `device`, which the kernels read by pointer, so no host
    synchronisation takes place (the reference keeps a traced device scalar).
    """
    if descale is None:
        return 1.0
    if isinstance(descale, (int, float)):
        return float(descale)
    t = as_tensor(descale)
    if t.numel() != 1:
        raise ValueError(f"{arg_name} must be one per-tensor value; got shape {tuple(t.shape)}.")
    return t.reshape(1).to(device=device, dtype=torch.float32)


def set_descales(params, k_descale, v_descale):
    """Fill the k/v descale fields of a DecodeParams / PrefillParams from
    descale_scalar's results (a float by value, a device tensor by pointer).
    Returns the tensors the launch reads, to be kept alive until it is
    enqueued."""
    keep = []
    for name, val in (("k_descale", k_descale), ("v_descale", v_descale)):
        if isinstance(val, torch.Tensor):
            setattr(params, name, 1.0)
            setattr(params, name + "_ptr", val.data_ptr())
            keep.append(val)
        else:
            setattr(params, name, float(val))
            setattr(params, name + "_ptr", None)
    return keep


def check_sinks(sinks, nheads, device):
    """`inputs.py:75-87`: (nheads,) float sink logits as f32 on device, or None."""
    if sinks is None:
        return None
    sinks = as_tensor(sinks)
    if tuple(sinks.shape) != (nheads,) or not sinks.is_floating_point():
        raise ValueError(
            f"learnable_sink must be a ({nheads},) float array, one logit per"
            f" query head; got {tuple(sinks.shape)} {sinks.dtype}."
        )
    return sinks.to(device=device, dtype=torch.float32).contiguous()


def resolve_scale(softmax_scale, head_dim):
    return 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)


def effective_window(causal, window_size):
    """`variant.py:205-217`: (left, right) with -1 unbounded; causal forces right 0."""
    left, right = window_size
    if causal:
        right = 0
    return left, right


def check_paged_window(causal, window_size):
    """`variant.py:232-240`: a paged cache takes a right bound of -1 or 0."""
    _, right = effective_window(causal, window_size)
    if right not in (-1, 0):
        raise NotImplementedError(
            "a paged KV cache takes a window right bound of -1 (unbounded)"
            f" or 0 (causal) only; got window_size={window_size}."
        )


def int32_device(x, device, name, shape=None):
    """An int32 contiguous device tensor from an int / array / tensor."""
    if isinstance(x, int):
        t = torch.tensor([x], dtype=torch.int32, device=device)
    else:
        t = as_tensor(x)
        if t.is_floating_point() or t.dtype == torch.bool:
            raise ValueError(f"{name} must be an integer array; got {t.dtype}.")
        t = t.to(device=device, dtype=torch.int32).contiguous()
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be {tuple(shape)}; got {tuple(t.shape)}.")
    return t
