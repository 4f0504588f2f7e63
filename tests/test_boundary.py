"""Host-side checks of the drop-in boundary that run without a GPU: the state-tuple checks
(the reference's layouts, models.py:1030-1056, with its int8 refractory counter, :574-583),
the workspace ledger behind ``V1Column.check_rollout``, and the ownership of the cell's one
fused voltage loss (``VoltageRegularization``)."""
import gc
import types

import pytest
import torch

from v1_glif_model_amd import losses
from v1_glif_model_amd.models import V1Column, WorkspaceLedger, _check_tensor


def _fake_cell(N=7, D=3, nb=4, r_dtype=torch.int8):
    return types.SimpleNamespace(_n_neurons=N, max_delay=D, _n_syn_basis=nb, device=torch.device("cpu"),
                                 _refractory_state_dtype=r_dtype)


def _state(B, N=7, D=3, nb=4, r_dtype=torch.int8):
    z = lambda *s: torch.zeros(s, dtype=torch.float32)
    return (z(B, N * D), z(B, N), torch.zeros((B, N), dtype=r_dtype), z(B, 2 * N), z(B, N * nb), z(B, N * nb),
            torch.zeros((B,), dtype=torch.int32))


def test_state_of_the_reference_layout_passes():
    cell = _fake_cell()
    V1Column.check_state(cell, _state(2), 2)
    V1Column.check_state(cell, _state(2, r_dtype=torch.int16), 2)
    V1Column.check_state(cell, _state(2)[:6], 2)


@pytest.mark.parametrize("i,bad", [
    (0, torch.zeros((2, 20))),                        # z_buf one column short
    (1, torch.zeros((3, 7))),                         # v of another batch size
    (2, torch.zeros((2, 7), dtype=torch.int32)),      # r neither int8 nor int16
    (2, torch.zeros((2, 7))),                         # r as float
    (3, torch.zeros((2, 7))),                         # asc [B, N] instead of [B, 2N]
    (4, torch.zeros((2, 28), dtype=torch.float64)),   # psc_rise in float64
    (5, "psc"),                                       # not a tensor
    (6, torch.zeros((2,), dtype=torch.float32)),      # noise_step as float
])
def test_state_with_a_wrong_tensor_raises(i, bad):
    st = list(_state(2))
    st[i] = bad
    with pytest.raises(ValueError):
        V1Column.check_state(_fake_cell(), st, 2)


def test_state_on_another_device_raises():
    cell = _fake_cell()
    cell.device = torch.device("cuda", 0)   # the CPU tensors are then on the wrong device
    with pytest.raises(ValueError, match="is on cpu"):
        V1Column.check_state(cell, _state(2), 2)


def test_int8_refractory_state_refused_when_periods_exceed_127_steps():
    with pytest.raises(ValueError, match="int16"):
        V1Column.check_state(_fake_cell(r_dtype=torch.int16), _state(2), 2)


def test_wrong_tuple_length_raises():
    with pytest.raises(ValueError):
        V1Column.check_state(_fake_cell(), _state(2)[:5], 2)


def test_in_place_buffers_must_be_contiguous():
    t = torch.zeros((4, 6), dtype=torch.int32).t()
    with pytest.raises(ValueError, match="contiguous"):
        _check_tensor(t, "spike_count", (6, 4), (torch.int32,), torch.device("cpu"), contiguous=True)


def test_ledger_keeps_any_number_of_pending_workspaces():
    """More pending rollouts than any fixed cap: every one is still recognised as the last
    writer of its own workspace, and an overwrite is still seen."""
    led = WorkspaceLedger()
    wss = [torch.empty(16, dtype=torch.uint8) for _ in range(200)]
    for g, ws in enumerate(wss, 1):
        led.record(ws, g)
    assert all(led.holds(ws, g) for g, ws in enumerate(wss, 1))
    led.record(wss[5], 1000)            # a later rollout on the same workspace
    assert not led.holds(wss[5], 6) and led.holds(wss[5], 1000)
    alias = wss[7].view(torch.uint8)    # another tensor object at the same address
    led.record(alias, 1001)
    assert not led.holds(wss[7], 8)


def test_ledger_forgets_a_freed_workspace_but_not_a_live_alias():
    led = WorkspaceLedger()
    a = torch.empty(64, dtype=torch.uint8)
    led.record(a, 1)
    assert len(led) == 1
    del a
    gc.collect()
    assert len(led) == 0
    b = torch.empty(64, dtype=torch.uint8)
    v = b[:]                            # same address, another object
    led.record(b, 2)
    led.record(v, 3)
    del b
    gc.collect()
    assert led.holds(v, 3)              # the entry belongs to the live alias


class _FakeLib:
    """Records the cell's fused voltage-loss settings as libglif would hold them."""

    def __init__(self):
        self.mode, self.cost, self.mask = 0, 0.0, None

    def glif_cell_set_voltage_loss(self, handle, mode, cost):
        self.mode, self.cost = mode, cost
        return 0

    def glif_cell_set_voltage_mask(self, handle, mask, n):
        self.mask = None if mask is None else (mask.value, n)
        return 0


def test_rebinding_a_regularizer_keeps_the_new_one_enabled(monkeypatch):
    """reg = VoltageRegularization(cell); reg = VoltageRegularization(cell): the first object's
    deletion runs after the second's constructor and must not switch the loss off."""
    fake = _FakeLib()
    monkeypatch.setattr(losses, "lib", lambda: fake)
    cell = types.SimpleNamespace(handle=object(), device=torch.device("cpu"), _n_neurons=6)
    reg = losses.VoltageRegularization(cell, voltage_cost=0.25, penalty_mode="threshold")
    assert (fake.mode, fake.cost) == (2, 0.25)
    reg = losses.VoltageRegularization(cell, voltage_cost=0.5, penalty_mode="range",
                                       core_mask=[1, 0, 1, 0, 0, 0])
    gc.collect()
    assert (fake.mode, fake.cost) == (1, 0.5) and fake.mask is not None and fake.mask[1] == 2
    assert reg._owns()
    # the tensor form hands its gradient to autograd: the fused one goes off
    reg(torch.zeros((2, 1, 6)))
    assert fake.mode == 0 and fake.mask is None
    # a third regularizer takes the loss; disabling the second leaves the third's on
    other = losses.VoltageRegularization(cell, voltage_cost=3.0, penalty_mode="threshold")
    reg.disable()
    assert (fake.mode, fake.cost) == (2, 3.0)
    del other
    gc.collect()
    assert fake.mode == 0


def test_a_fused_call_reclaims_the_loss(monkeypatch):
    fake = _FakeLib()
    monkeypatch.setattr(losses, "lib", lambda: fake)
    cell = types.SimpleNamespace(handle=object(), device=torch.device("cpu"), _n_neurons=4)
    a = losses.VoltageRegularization(cell, voltage_cost=1.0, penalty_mode="range", core_mask=[1, 1, 0, 0])
    b = losses.VoltageRegularization(cell, voltage_cost=2.0, penalty_mode="threshold")
    assert (fake.mode, fake.cost, fake.mask) == (2, 2.0, None)
    cell.check_rollout = lambda: (_ for _ in ()).throw(RuntimeError("stop after claiming"))
    with pytest.raises(RuntimeError, match="stop after claiming"):
        a()                              # fused: a claims the loss back, with its own mask
    assert (fake.mode, fake.cost) == (1, 1.0) and fake.mask[1] == 2
    assert a._owns() and not b._owns()
    del b
    gc.collect()
    assert fake.mode == 1                # b no longer owned it
