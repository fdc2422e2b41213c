"""Helpers shared by the stack tests: the oracle's view of the stack's weights and state."""
import torch


def _bank(b):
    return (b.packed.cpu(), b.scales.cpu(), b.group_size)


def oracle_layer_weights(lw) -> dict:
    """``target.LayerWeights`` (portable banks, any device) -> the dict ``oracle.stack`` reads."""
    d = {"kind": lw.kind, "input_norm": lw.input_norm.cpu(), "post_norm": lw.post_norm.cpu(),
         "mixer_in": _bank(lw.mixer_in), "mixer_out": _bank(lw.mixer_out), "router": lw.router.cpu(),
         "gate_up": _bank(lw.gate_up), "down": _bank(lw.down),
         "shared": (_bank(lw.shared.gate_up), _bank(lw.shared.down), lw.shared.gate_weight.cpu())}
    for name in ("conv", "a_log", "dt_bias", "gdn_norm", "q_norm", "k_norm"):
        v = getattr(lw, name)
        if v is not None:
            d[name] = v.cpu()
    return d


def oracle_layer_state(state, i: int) -> dict:
    """Layer ``i`` of a ``target.TargetState`` as CPU tensors."""
    if state.keys[i] is not None:
        return {"keys": state.keys[i][0].cpu(), "values": state.values[i][0].cpu()}
    return {"conv": state.conv[i][0].cpu(), "recurrent": state.recurrent[i].cpu()}
