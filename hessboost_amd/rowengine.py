"""A Python host of hessboost's device-resident round over the row engine
of the C ABI: the caller's side of the RowEngine seam, call for call as the
reference's Rust builder issues it, for hosts without the Rust shim.

`RowEngineRounds.device_round` follows src/training/round.rs:105-148:
margins loaded once, the gradients computed on the device, one tree grown
as `build_device_staged` grows it (src/tree/builder/hist/device.rs:233-247
-> build_on_device :147-231, grow_device_depthwise :249-294,
resident_children :441-528, resident_search/resident_merge :530-627,
resident_best :650-700), the leaves scaled by eta and added to the margins
by their segments. Depthwise growth, no column sampling, no monotone
constraints. The host arithmetic the reference performs between the calls
(node gains, leaf weights) comes from the library (hbr_node_gain,
hbr_leaf_weight). The sums are fixed point with the guard resolving near
ties on the device (HBR_GUARD_RESOLVE), so no node comes back for a host
replay; one that does (a NaN score) stops the round with an error, the
reference's `None`: the caller redoes the round on its own path.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np

from . import _capi as A

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


class RowEngineRounds:
    """Depthwise logistic or squared-error rounds over one engine (dense
    index), driven through hbr_* row-engine calls."""

    def __init__(self, engine, feature_offset, cut_values, params: dict, loss=A.LOSS_LOGISTIC):
        self.e = engine
        self.fo = np.asarray(feature_offset, np.int64)
        self.cuts = np.asarray(cut_values, np.float32)
        self.max_depth = params.get("max_depth", 6)
        self.eta = np.float32(params.get("eta", params.get("learning_rate", 0.3)))
        self.gamma = float(params.get("gamma", 0.0))
        self.mcw = float(params.get("min_child_weight", 1.0))
        self.reg = (params.get("lambda", 1.0), params.get("alpha", 0.0), params.get("max_delta_step", 0.0), self.mcw)
        self._rp = A.RegParams(*self.reg)
        self.loss = loss
        self.replays = 0
        self.audit = None  # a list: every certified numeric winner with read_hist's sums of its node
        self.margins_loaded = False
        engine.set_guard("resolve", self.gamma)

    # ---- host arithmetic (the reference's builder, through the library) --------
    def node_gain(self, st, lower=-math.inf, upper=math.inf):
        out = C.c_float()
        A.check(A.lib().hbr_node_gain(C.byref(self._rp), st.g, st.h, lower, upper, C.byref(out)))
        return out.value

    def valid(self, b):
        """BestSplit::valid (builder/mod.rs:167-193)."""
        lh, rh = b.left.h, b.right.h
        return (b.loss_chg > 1e-6 and b.loss_chg >= self.gamma and lh > 0.0 and rh > 0.0 and lh >= self.mcw
                and rh >= self.mcw)

    def leaf_value(self, st):
        out = C.c_float()
        A.check(A.lib().hbr_leaf_weight(C.byref(self._rp), st.g, st.h, -math.inf, math.inf, C.byref(out)))
        return np.float32(np.float32(out.value) * self.eta)

    # ---- resident search (device.rs:530-700) -------------------------------------
    def search(self, nodes):
        """nodes: [(slot, Stats)] -> [Best]."""
        reqs = [dict(slot=slot, total=(st.g, st.h), fixed=st.fixed, root_gain=self.node_gain(st))
                for slot, st in nodes]
        scans = self.e.scan_resident(self.reg, reqs)
        out = []
        for (slot, st), sc in zip(nodes, scans):
            if sc.kind == A.SCAN_REPLAY:
                # NodeScan::Replay (a NaN score): this host has no search of its own
                self.replays += 1
                raise RuntimeError(f"row engine: node in slot {slot} needs a host replay (reason {sc.fallback})")
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
                self.audit.append(dict(slot=slot, total=(st.g, st.h), feature=sc.feature, bin=b.bin,
                                       default_left=b.default_left, loss=sc.loss_chg, err=sc.loss_err,
                                       hist=self.e.read_hist(slot)))
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
        if not e.reserve_hists(reserved):
            raise RuntimeError("row engine: the histogram slots do not fit")
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
        if not e.gradients(self.loss, labels):
            raise RuntimeError("row engine: non-finite gradients (the reference grows this round on the host)")
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
