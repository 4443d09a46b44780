"""Host logic of the epoch-free batcher's scheduler (no GPU): admission in
arrival order up to max_rows, finished and cancelled rows leave before the
next step and their places are refilled at once (the reference refills only
at an epoch boundary, ContinuousBatcher.swift:277-301, :455-458)."""
import pytest

from krill_amd.batcher import Request, Scheduler


def _ids(rows):
    return [r.req.rid for r in rows]


def test_admits_in_arrival_order_up_to_max_rows():
    s = Scheduler(2)
    for i in range(4):
        s.submit(Request(i, 10, 3))
    retired, admitted = s.plan_step()
    assert retired == [] and _ids(admitted) == [0, 1] and _ids(s.rows) == [0, 1]
    retired, admitted = s.plan_step()
    assert retired == [] and admitted == []


def test_finished_row_is_replaced_in_the_same_step():
    s = Scheduler(2)
    for i in range(3):
        s.submit(Request(i, 10, 3))
    s.plan_step()
    s.rows[0].finished = True
    retired, admitted = s.plan_step()
    assert _ids(retired) == [0] and _ids(admitted) == [2]
    assert _ids(s.rows) == [1, 2]  # the running row keeps its place, the newcomer joins at the end


def test_cancel_running_and_pending():
    s = Scheduler(2)
    for i in range(4):
        s.submit(Request(i, 10, 3))
    s.plan_step()
    s.cancel(1)  # running
    s.cancel(2)  # pending: never admitted
    retired, admitted = s.plan_step()
    assert _ids(retired) == [1] and _ids(admitted) == [3] and _ids(s.rows) == [0, 3]
    for r in s.rows:
        r.finished = True
    s.plan_step()
    assert s.idle


def test_rejects_bad_requests():
    with pytest.raises(ValueError):
        Scheduler(0)
    s = Scheduler(1)
    with pytest.raises(ValueError):
        s.submit(Request(0, 0, 1))
