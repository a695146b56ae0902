"""The oracle's user-UpdateConn pass (oracle/growth.py update_conn), pinned by
the known answers of the reference's tests/test_update_conn.py."""

from __future__ import annotations

import numpy as np

import nets
import update_conn_cases as uc


def _step(oracle, net, static, state):
    o = nets.oracle_for(oracle, net, static, state)
    o.step(np.zeros(len(static.input_ids), np.float32))
    return o


def test_incoming_and_outgoing_bind_their_endpoints(oracle) -> None:
    for cls in (uc.IncomingEndpoint, uc.OutgoingEndpoint):
        static, state = uc.endpoint_probe(cls, "cpu")
        o = _step(oracle, uc.net(cls()), static, state)
        w, dead = o.conns[0]["weight"], o.conns[0]["dead"].astype(bool)
        assert sorted(w[~dead].tolist()) == [80.0, 90.0]


def test_outgoing_reads_incoming_writes_in_every_bucket_and_dead_slots_keep_theirs(oracle) -> None:
    static, state = uc.order_probe_topological("cpu")
    assert len(static.level_capacities) == 3
    o = _step(oracle, uc.net(uc.OrderProbe(), uc.px.Propagation.TOPOLOGICAL), static, state)
    for b, bucket in enumerate(o.conns):
        dead = bucket["dead"].astype(bool)
        assert (~dead).any()
        assert (bucket["weight"][~dead] == np.float32(uc.INCOMING_MARK + 1000.0)).all(), b
        assert (bucket["weight"][dead] == 0.0).all(), b  # the column default, untouched
