"""hessboost's device-resident round, driven call for call through the row
engine of the C ABI, as the reference issues it (test harness).

`device_round` follows src/training/round.rs:105-148: margins loaded once,
the gradients computed on the device, one tree grown by
`build_device_staged` (src/tree/builder/hist/device.rs:233-247 ->
build_on_device :147-231, grow_device_depthwise :249-294,
resident_children :441-528, resident_search/resident_merge :530-627,
resident_best :650-700), the leaves scaled by eta and added to the margins
by their segments. The host-side arithmetic the reference performs between
the calls (node gains, validity, leaf weights) comes from the oracle, which
restates the reference's CPU builder; a replayed node (NodeScan::Replay) is
evaluated by the oracle on the histogram hbr_read_hist returns, as
resident_merge evaluates it on the host.
"""
from __future__ import annotations

import math

import numpy as np

from hessboost_amd import _capi as A
from oracle import oracle as O

F32_MAX = float(np.finfo(np.float32).max)


class Stats:
    __slots__ = ("g", "h", "fixed")

    def __init__(self, g, h, fixed=None):
        self.g, self.h, self.fixed = float(g), float(h), fixed


class Best:
    """A node's winner as the host records it (BestSplit)."""

    def __init__(self, loss_chg=0.0, feature=0, bin_=-1, default_left=True, left=None, right=None, valid_split=False):
        self.loss_chg, self.feature, self.bin, self.default_left = loss_chg, feature, bin_, default_left
        self.left, self.right, self.valid_split = left, right, valid_split


class Driver:
    """One engine over a dense index, driven through hbr_* row-engine calls."""

    def __init__(self, engine, cuts_fo, cut_values, params: dict):
        self.e = engine
        self.fo = np.asarray(cuts_fo, np.int64)
        self.cuts = np.asarray(cut_values, np.float32)
        self.max_depth = params.get("max_depth", 6)
        self.eta = np.float32(params.get("eta", 0.3))
        self.p = O.params(objective=O.OBJ_LOGISTIC, max_depth=self.max_depth, eta=float(self.eta),
                          gamma=params.get("gamma", 0.0), reg_lambda=params.get("lambda", 1.0),
                          min_child_weight=params.get("min_child_weight", 1.0))
        self.reg = (params.get("lambda", 1.0), 0.0, 0.0, params.get("min_child_weight", 1.0))
        self.replays = 0
        self.audit = None  # a list: every certified numeric winner with the host's evaluation of its exact sums
        self.margins_loaded = False
        self.ds = None  # the oracle's index, for replays (set by the caller)

    # ---- host arithmetic (the reference's builder, as the oracle restates it) ----
    def node_gain(self, st, lower=-math.inf, upper=math.inf):
        return O.lib().or_node_gain(st.g, st.h, lower, upper, self.p)

    def valid(self, b: Best):
        s = O.Split()
        s.loss_chg, s.left_h, s.right_h = b.loss_chg, b.left.h, b.right.h
        return bool(O.lib().or_split_valid(s, self.p))

    def leaf_value(self, st):
        w = np.float32(O.lib().or_calc_weight(st.g, st.h, self.p))
        return np.float32(w * self.eta)

    # ---- resident search (device.rs:530-700) -------------------------------------
    def search(self, nodes):
        """nodes: [(slot, Stats)] -> [Best]."""
        reqs = [dict(slot=slot, total=(st.g, st.h), fixed=st.fixed, root_gain=self.node_gain(st))
                for slot, st in nodes]
        scans = self.e.scan_resident(self.reg, reqs)
        out = []
        for (slot, st), sc in zip(nodes, scans):
            if sc.kind == A.SCAN_REPLAY:
                # resident_merge: the node's histogram, evaluated on the host
                self.replays += 1
                hist = self.e.read_hist(slot)
                s = self.ds.evaluate(hist, (st.g, st.h), self.p)
                b = Best(s.loss_chg, s.feature, s.bin, bool(s.default_left), Stats(s.left_g, s.left_h),
                         Stats(s.right_g, s.right_h))
            elif sc.kind == A.SCAN_EMPTY:
                b = Best()
            else:
                first = int(self.fo[sc.feature])
                acc = Stats(sc.acc_g, sc.acc_h)
                rest = Stats(st.g - sc.acc_g, st.h - sc.acc_h)
                if sc.backward:
                    # SplitPos::backward(first, offset): bins below offset go left
                    bin_ = first + sc.offset - 1 if sc.offset > 0 else -1
                    left, right = rest, acc
                    left.fixed = (sc.fixed_left_g, sc.fixed_left_h)
                    right.fixed = (sc.fixed_right_g, sc.fixed_right_h)
                    b = Best(float(np.float32(sc.loss_chg)), sc.feature, bin_, True, left, right)
                else:
                    left, right = acc, rest
                    left.fixed = (sc.fixed_left_g, sc.fixed_left_h)
                    right.fixed = (sc.fixed_right_g, sc.fixed_right_h)
                    b = Best(float(np.float32(sc.loss_chg)), sc.feature, first + sc.offset, False, left, right)
            if b.left is not None:
                b.valid_split = self.valid(b)
            if self.audit is not None and sc.kind == A.SCAN_NUMERIC:
                exact = self.ds.evaluate(self.e.read_hist(slot), (st.g, st.h), self.p)
                self.audit.append((sc.feature, b.bin, b.default_left, sc.loss_chg, sc.loss_err, exact))
            out.append(b)
        return out

    # ---- one tree (build_on_device, grow_device_depthwise) -----------------------
    def grow(self):
        e = self.e
        root_seg = e.begin_tree()
        tot, fx = e.root_total(root_seg, fixed=True)
        root = Stats(tot[0], tot[1], (int(fx[0]), int(fx[1])))
        n_rows = int(root_seg.len)
        reserved = min(1 << (self.max_depth - 1), max(n_rows, 1))
        assert e.reserve_hists(reserved)
        free, next_slot = [], [0]

        def take():
            if free:
                return free.pop()
            s = next_slot[0]
            next_slot[0] += 1
            assert s < reserved
            return s

        slot = take()
        e.build_resident([(root_seg, slot)])
        best = self.search([(slot, root)])[0]
        # tree nodes: dicts as compare_trees reads them
        nodes = [dict(left=-1, right=-1, split_feature=0, split_cond=0.0, default_left=True, leaf_value=0.0)]
        frontier = [(0, root_seg, slot, root, best)]
        leaves = []  # (node id, segment, stats)
        depth = 0
        while depth < self.max_depth and frontier:
            pending = []
            for nid, seg, sl, st, b in frontier:
                if b.left is not None and b.valid_split:
                    left_id = len(nodes)
                    nd = nodes[nid]
                    nd.update(left=left_id, right=left_id + 1, split_feature=b.feature, default_left=b.default_left,
                              split_cond=float(self.cuts[b.bin]) if b.bin >= 0 else -F32_MAX)
                    nodes.append(dict(left=-1, right=-1, split_feature=0, split_cond=0.0, default_left=True,
                                      leaf_value=0.0))
                    nodes.append(dict(left=-1, right=-1, split_feature=0, split_cond=0.0, default_left=True,
                                      leaf_value=0.0))
                    terminal = depth + 1 >= self.max_depth
                    pending.append((nid, seg, sl, b, left_id, terminal))
                else:
                    free.append(sl)
                    leaves.append((nid, seg, st))
            if not pending:
                frontier = []
                break
            # partition_pending: one device partition of every split, in order
            splits = []
            for nid, seg, sl, b, left_id, terminal in pending:
                first = int(self.fo[b.feature])
                limit = b.bin + 1 - first if b.bin >= 0 else 0
                splits.append((seg, b.feature, limit, b.default_left))
            parts = e.partition(splits)
            # resident_children
            for nid, seg, sl, b, left_id, terminal in pending:
                if terminal:
                    free.append(sl)
            build, siblings, child_slots = [], [], []
            for (nid, seg, sl, b, left_id, terminal), (lseg, rseg) in zip(pending, parts):
                if terminal:
                    child_slots.append(None)
                    continue
                built = take()
                left_smaller = lseg.len <= rseg.len
                build.append((lseg if left_smaller else rseg, built))
                siblings.append((sl, built))
                child_slots.append((built, sl) if left_smaller else (sl, built))
            if build:
                e.build_resident(build, siblings)
            requests = []
            for (nid, seg, sl, b, left_id, terminal), cs in zip(pending, child_slots):
                if cs is not None:
                    requests.append((cs[0], b.left))
                    requests.append((cs[1], b.right))
            bests = iter(self.search(requests)) if requests else iter(())
            frontier = []
            for (nid, seg, sl, b, left_id, terminal), cs, (lseg, rseg) in zip(pending, child_slots, parts):
                if cs is None:
                    leaves.append((left_id, lseg, b.left))
                    leaves.append((left_id + 1, rseg, b.right))
                else:
                    frontier.append((left_id, lseg, cs[0], b.left, next(bests)))
                    frontier.append((left_id + 1, rseg, cs[1], b.right, next(bests)))
            depth += 1
        for nid, seg, sl, st, b in frontier:
            leaves.append((nid, seg, st))
        for nid, seg, st in leaves:
            nodes[nid]["leaf_value"] = self.leaf_value(st)
        return nodes, leaves

    # ---- the round (round.rs:105-148) --------------------------------------------
    def device_round(self, margins, labels):
        e = self.e
        if not self.margins_loaded:
            e.load_margins(margins)
            self.margins_loaded = True
        assert e.gradients(A.LOSS_LOGISTIC, labels)
        nodes, leaves = self.grow()
        e.add_leaf_values([seg for _, seg, _ in leaves], [nodes[nid]["leaf_value"] for nid, _, _ in leaves])
        return nodes


def as_tree(nodes):
    """The driver's nodes as the column dict compare_trees reads."""
    return dict(left=np.array([n["left"] for n in nodes], np.int32), right=np.array([n["right"] for n in nodes], np.int32),
                split_feature=np.array([n["split_feature"] for n in nodes], np.uint32),
                split_cond=np.array([n["split_cond"] for n in nodes], np.float32),
                default_left=np.array([n["default_left"] for n in nodes], np.uint8),
                leaf_value=np.array([n["leaf_value"] for n in nodes], np.float32))
