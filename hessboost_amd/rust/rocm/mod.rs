//! The AMD MI355X (gfx950) backend (Linux, `rocm` feature): hessboost's
//! histogram and row-engine traits over `libhbrocm.so`.
//!
//! This module is written for hessboost's crate tree, where it sits beside
//! the CUDA backend as `src/backend/rocm/` (`mod.rs`, `ffi.rs`,
//! `predict.rs`), declared in `src/backend/mod.rs` as
//! `#[cfg(all(target_os = "linux", feature = "rocm"))] pub mod rocm;`.
//!
//! **Training** (`device = rocm` / `rocm:<ordinal>`): [`RocmHistBackend`]
//! implements [`HistogramBackend`] (src/tree/hist/mod.rs:73-105) and
//! [`RowEngine`] (src/tree/hist/mod.rs:213-295). The engine keeps the index,
//! the staged gradient pairs, a tree's rows and the resident histograms on
//! the GPU; each trait call is one library call. Histograms are summed in
//! fixed point (exact integers in a per-tree unit): inside the exact domain
//! of `backend/exact_sum.rs:14-37` they are the CPU's `f64` sums bit for
//! bit. Beyond it the training parameter `rocm_sums` ([`RocmSums`]) decides:
//! `fixed_point` (the default for `device = rocm`) keeps every round on the
//! device with the fixed-point sums, each split certified by the library's
//! guard against the CPU's `f64` sums and any node it cannot certify
//! searched again on the device over the node's histogram in the CPU
//! builder's own summation order; `exact` makes the library refuse
//! (`HBR_REFUSED`) and this module sum on the host, as `CudaHistBackend`
//! does outside its exact domain (src/backend/cuda/mod.rs:2758-2776).
//!
//! **Prediction**: [`RocmModel`] ([`BoostedModel::to_rocm`]) uploads the
//! forest once; margins are walked on the GPU, the objective's transform
//! runs on the CPU.
//!
//! Status mapping: `HBR_OK` is `Some`, `HBR_REFUSED` and `HBR_INVALID` are
//! `None` (the builder then does the work on the host), `HBR_DEVICE_ERROR`
//! is `None` plus the sticky `failed` flag, after which [`row_engine`]
//! returns `None` and every build runs on the CPU, as
//! src/backend/cuda/mod.rs:1806-1826 does for CUDA.
//!
//! [`row_engine`]: HistogramBackend::row_engine

mod ffi;
mod predict;

pub use predict::RocmModel;

use crate::data::ghist::{Bins, GHistIndex};
use crate::error::{HessboostError, Result};
use crate::objective::GradPair;
use crate::tree::gain::{GradStats, RegParams};
use crate::tree::hist::{
    CpuBackend, DeviceLoss, HistSlot, Histogram, HistogramBackend, NodeScan, Partitioned, RowEngine, RowRule,
    RowSplit, ScanFallback, ScanRequest, Segment,
};
use std::os::raw::{c_char, c_int};
use std::ptr::{self, NonNull};
use std::sync::atomic::{AtomicBool, Ordering};
use std::sync::{Mutex, MutexGuard};

// `ghist.row_ptr()` (usize) is handed to the library as u64.
const _: () = assert!(std::mem::size_of::<usize>() == 8);
// `out: &mut [GradStats]` is written as interleaved f64 (g, h).
const _: () = assert!(std::mem::size_of::<GradStats>() == 16);
// `&[GradPair]` is read as interleaved f32 (g, h).
const _: () = assert!(std::mem::size_of::<GradPair>() == 8);

/// The lanes of the host's logistic vector kernel the device restates
/// (`simd/x86_64.rs:22-51`, eight f32 lanes); other splits run on the host.
const DEVICE_VECTOR_LANES: usize = 8;

/// The calling thread's last message from the library.
pub(crate) fn last_error() -> String {
    let mut buf = vec![0u8; 256];
    // SAFETY: the library writes at most `len` bytes, terminator included.
    let full = unsafe { ffi::hbr_last_error(buf.as_mut_ptr().cast::<c_char>(), buf.len()) };
    if full >= buf.len() {
        buf.resize(full + 1, 0);
        // SAFETY: as above, with room for the whole message.
        unsafe { ffi::hbr_last_error(buf.as_mut_ptr().cast::<c_char>(), buf.len()) };
    }
    buf.truncate(full);
    String::from_utf8_lossy(&buf).into_owned()
}

/// A failed call as the crate's error (constructors and prediction, which
/// return `Result`).
pub(crate) fn check(status: c_int) -> Result<()> {
    match status {
        ffi::HBR_OK => Ok(()),
        _ => Err(HessboostError::gpu(format!("rocm: {}", last_error()))),
    }
}

/// Number of ROCm devices visible to the process (0 when the runtime is
/// absent).
pub fn device_count() -> usize {
    let mut n: c_int = 0;
    // SAFETY: writes one int.
    match unsafe { ffi::hbr_device_count(&mut n) } {
        ffi::HBR_OK => n.max(0) as usize,
        _ => 0,
    }
}

/// Whether `device = rocm:<ordinal>` can run (the parameter validation's
/// check, beside CUDA's `available`).
pub fn available(ordinal: usize) -> bool {
    ordinal < device_count()
}

/// The name and architecture of ROCm device `ordinal`, if it exists.
pub fn device_name(ordinal: usize) -> Option<String> {
    let ordinal = c_int::try_from(ordinal).ok()?;
    let mut buf = [0 as c_char; 256];
    // SAFETY: the buffer's length bounds the write, NUL included.
    if unsafe { ffi::hbr_device_name(ordinal, buf.as_mut_ptr(), buf.len()) } != ffi::HBR_OK {
        return None;
    }
    // SAFETY: NUL-terminated within the buffer.
    Some(unsafe { std::ffi::CStr::from_ptr(buf.as_ptr()) }.to_string_lossy().into_owned())
}

/// The gradient slice [`HistogramBackend::prepare`] staged, by address and
/// length: a `build` of the same slice reads what the device holds.
#[derive(Clone, Copy, PartialEq, Eq)]
struct StagedSlice {
    ptr: usize,
    len: usize,
}

impl StagedSlice {
    fn of(gpair: &[GradPair]) -> Self {
        Self {
            ptr: gpair.as_ptr() as usize,
            len: gpair.len(),
        }
    }
}

/// How the backend sums beyond the exact domain (the training parameter
/// `rocm_sums`, `fixed_point` or `exact`).
#[derive(Debug, Clone, Copy, PartialEq, Eq, Default)]
pub enum RocmSums {
    /// Fixed-point sums on the device, every split certified against the
    /// CPU's `f64` sums (near ties resolved on the device's copy of those
    /// sums): whole rounds stay on the GPU. Tree structure equals the CPU's;
    /// leaf values and statistics are within the fixed point's error (the
    /// north star's 1e-5 relative).
    #[default]
    FixedPoint,
    /// Only sums equal to the CPU's bit for bit: the library refuses beyond
    /// the exact domain and the host sums, as the CUDA backend does.
    Exact,
}

impl RocmSums {
    /// The parameter's spellings.
    pub fn parse(value: &str) -> Option<Self> {
        match value {
            "fixed_point" => Some(Self::FixedPoint),
            "exact" => Some(Self::Exact),
            _ => None,
        }
    }
}

/// hessboost's histogram backend and row engine on one MI355X GPU.
pub struct RocmHistBackend {
    engine: NonNull<ffi::hbr_engine>,
    ordinal: usize,
    /// The index the engine was opened on (`GHistIndex::identity`,
    /// src/data/ghist.rs:260, compiled for `rocm` as for `cuda`).
    identity: u64,
    n_rows: usize,
    n_cols: usize,
    total_bins: usize,
    failed: AtomicBool,
    staged: Mutex<Option<StagedSlice>>,
}

// SAFETY: the library serializes every call on a handle behind the
// handle's own mutex and never calls back; the handle is freed once, in
// `Drop`.
unsafe impl Send for RocmHistBackend {}
// SAFETY: as above.
unsafe impl Sync for RocmHistBackend {}

impl std::fmt::Debug for RocmHistBackend {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        f.debug_struct("RocmHistBackend")
            .field("ordinal", &self.ordinal)
            .field("n_rows", &self.n_rows)
            .field("n_cols", &self.n_cols)
            .field("total_bins", &self.total_bins)
            .field("failed", &self.failed.load(Ordering::Relaxed))
            .finish_non_exhaustive()
    }
}

impl Drop for RocmHistBackend {
    fn drop(&mut self) {
        // SAFETY: opened by `hbr_engine_open*`, closed exactly once.
        unsafe { ffi::hbr_engine_close(self.engine.as_ptr()) }
    }
}

impl RocmHistBackend {
    /// Upload `index` to ROCm device `ordinal` (the constructor
    /// `CudaHistBackend::new`, src/backend/cuda/mod.rs:1626-1671, mirrors):
    /// the row store as the reference lays it out (src/data/ghist.rs:195-209)
    /// plus the cuts and the categorical flags; the library re-encodes the
    /// rows on the device (dense u8 rows when every feature has at most 256
    /// bins, else CSR global bins).
    pub fn new(index: &GHistIndex, ordinal: usize) -> Result<Self> {
        let cuts = index.cuts();
        let n_cols = index.n_cols();
        let mut feature_offset = Vec::with_capacity(n_cols + 1);
        feature_offset.push(0u32);
        let mut cut_values = Vec::with_capacity(index.total_bins());
        let mut categorical = Vec::with_capacity(n_cols);
        for f in 0..n_cols {
            let (start, end) = cuts.feature_bins(f);
            cut_values.extend((start..end).map(|b| cuts.cut_value(b)));
            feature_offset.push(u32::try_from(end).map_err(|_| {
                HessboostError::invalid_data("index", "rocm: more than 2^32 bins")
            })?);
            categorical.push(u8::from(cuts.is_categorical(f)));
        }
        let (row_bins, row_bin_width) = match index.bins() {
            Bins::U16(bins) => (bins.as_ptr().cast(), 2u32),
            Bins::U32(bins) => (bins.as_ptr().cast(), 4u32),
        };
        let desc = ffi::hbr_index_desc {
            n_rows: index.n_rows() as u64,
            n_cols: n_cols as u64,
            feature_offset: feature_offset.as_ptr(),
            cut_values: cut_values.as_ptr(),
            row_ptr: index.row_ptr().as_ptr().cast::<u64>(),
            row_bins,
            row_bin_width,
            dense: u32::from(index.is_dense()),
            col_bins: ptr::null(),
            col_bin_width: 0,
            pad: 0,
            missing: ptr::null(),
            is_categorical: categorical.as_ptr(),
        };
        let mut engine = ptr::null_mut();
        let ordinal_c = c_int::try_from(ordinal)
            .map_err(|_| HessboostError::invalid_param("device", "rocm ordinal out of range"))?;
        // SAFETY: every pointer in `desc` outlives the call; the library
        // copies what it keeps.
        check(unsafe { ffi::hbr_engine_open(ordinal_c, &desc, &mut engine) })?;
        let engine = NonNull::new(engine).ok_or_else(|| HessboostError::gpu("rocm: no engine"))?;
        Ok(Self {
            engine,
            ordinal,
            identity: index.identity(),
            n_rows: index.n_rows(),
            n_cols,
            total_bins: index.total_bins(),
            failed: AtomicBool::new(false),
            staged: Mutex::new(None),
        })
    }

    /// The summing mode of a training run (`rocm_sums`) and its `gamma`
    /// (`min_split_loss`), the validity threshold the guard checks: fixed
    /// point selects `HBR_SUMS_FIXED_POINT` with the guard resolving near ties
    /// on the device (`HBR_GUARD_RESOLVE`); exact keeps `HBR_SUMS_EXACT`.
    pub fn with_sums(self, sums: RocmSums, gamma: f64) -> Result<Self> {
        let mode = match sums {
            RocmSums::FixedPoint => ffi::HBR_SUMS_FIXED_POINT,
            RocmSums::Exact => ffi::HBR_SUMS_EXACT,
        };
        // SAFETY: a live handle; plain values.
        check(unsafe { ffi::hbr_engine_set_sums(self.e(), mode) })?;
        check(unsafe { ffi::hbr_engine_set_guard(self.e(), ffi::HBR_GUARD_RESOLVE, gamma) })?;
        Ok(self)
    }

    /// The CUDA device ordinal's counterpart: the ROCm device this backend
    /// runs on.
    pub fn ordinal(&self) -> usize {
        self.ordinal
    }

    fn e(&self) -> *mut ffi::hbr_engine {
        self.engine.as_ptr()
    }

    fn staged(&self) -> MutexGuard<'_, Option<StagedSlice>> {
        self.staged.lock().unwrap_or_else(std::sync::PoisonError::into_inner)
    }

    /// One library status as the traits' `Option`.
    fn ok(&self, status: c_int) -> Option<()> {
        match status {
            ffi::HBR_OK => Some(()),
            ffi::HBR_DEVICE_ERROR => {
                self.failed.store(true, Ordering::Release);
                None
            }
            _ => None,
        }
    }

    fn fits(&self, ghist: &GHistIndex) -> bool {
        !self.failed.load(Ordering::Acquire) && ghist.identity() == self.identity
    }

    // ---- segments --------------------------------------------------------
    //
    // The engine keeps a tree's rows in two buffers of n_rows ids; a segment
    // is (buffer, offset, len). `Segment` records one offset, so the buffer
    // rides in it: offset = buffer * (n_rows + 1) + position.

    fn issue(&self, s: &ffi::hbr_segment) -> Segment {
        let offset = s.buffer as usize * (self.n_rows + 1) + s.offset as usize;
        Segment::issue(offset, s.len as usize, s.contiguous != 0, s.tree)
    }

    fn raw(&self, seg: &Segment) -> ffi::hbr_segment {
        let stride = self.n_rows + 1;
        ffi::hbr_segment {
            offset: (seg.offset() % stride) as u64,
            len: seg.len() as u64,
            buffer: (seg.offset() / stride) as u32,
            contiguous: u32::from(seg.contiguous()),
            tree: seg.tree(),
        }
    }

    /// The staged gradients, read back (the host copy a refused sum needs
    /// when the caller holds none).
    fn device_gradients(&self) -> Option<Vec<GradPair>> {
        let mut out = vec![GradPair::default(); self.n_rows];
        // SAFETY: n_rows pairs of f32.
        self.ok(unsafe { ffi::hbr_read_gradients(self.e(), out.as_mut_ptr().cast::<f32>(), self.n_rows as u64) })?;
        Some(out)
    }

    fn segment_rows(&self, seg: &Segment) -> Option<Vec<u32>> {
        let raw = self.raw(seg);
        let mut out = vec![0u32; seg.len()];
        // SAFETY: `len` ids.
        self.ok(unsafe { ffi::hbr_rows(self.e(), &raw, out.as_mut_ptr()) })?;
        Some(out)
    }

    /// A node's histogram summed on the host (`CpuBackend::build`) from its
    /// rows, for sums outside the exact domain.
    fn host_histogram(&self, ghist: &GHistIndex, gpair: &[GradPair], seg: &Segment) -> Option<Histogram> {
        let rows = self.segment_rows(seg)?;
        let mut out = vec![GradStats::default(); self.total_bins];
        CpuBackend.build(ghist, &rows, gpair, &mut out);
        Some(out)
    }
}

impl HistogramBackend for RocmHistBackend {
    fn build(&self, ghist: &GHistIndex, rows: &[u32], gpair: &[GradPair], out: &mut [GradStats]) {
        let on_device = self.fits(ghist)
            && out.len() == self.total_bins
            && gpair.len() == self.n_rows
            && rows.len() <= self.n_rows
            && rows.windows(2).all(|w| w[0] < w[1])
            && {
                let mut staged = self.staged();
                if *staged != Some(StagedSlice::of(gpair)) {
                    // SAFETY: n_rows interleaved (g, h) f32 pairs.
                    let st = unsafe { ffi::hbr_prepare(self.e(), gpair.as_ptr().cast(), gpair.len() as u64) };
                    *staged = self.ok(st).map(|()| StagedSlice::of(gpair));
                }
                staged.is_some()
            }
            && self
                .ok(unsafe {
                    // SAFETY: `rows` ids below n_rows; `out` holds total_bins
                    // (f64, f64) records, overwritten.
                    ffi::hbr_build(self.e(), rows.as_ptr(), rows.len() as u64, out.as_mut_ptr().cast::<f64>())
                })
                .is_some();
        if !on_device {
            CpuBackend.build(ghist, rows, gpair, out);
        }
    }

    fn prepare(&self, ghist: &GHistIndex, gpair: &[GradPair]) {
        let mut staged = self.staged();
        *staged = None;
        if !self.fits(ghist) || gpair.len() != self.n_rows {
            return;
        }
        // SAFETY: n_rows interleaved (g, h) f32 pairs, copied before return.
        let st = unsafe { ffi::hbr_prepare(self.e(), gpair.as_ptr().cast(), gpair.len() as u64) };
        *staged = self.ok(st).map(|()| StagedSlice::of(gpair));
    }

    fn row_engine(&self) -> Option<&dyn RowEngine> {
        (!self.failed.load(Ordering::Acquire)).then_some(self as &dyn RowEngine)
    }
}

impl RowEngine for RocmHistBackend {
    fn begin_tree(&self, ghist: &GHistIndex, rows: &[u32]) -> Option<Segment> {
        // the engine grows unsampled trees: every row, in order
        if !self.fits(ghist) || rows.len() != self.n_rows || !rows.iter().enumerate().all(|(i, &r)| r as usize == i)
        {
            return None;
        }
        let mut root = ffi::hbr_segment::default();
        // SAFETY: writes one segment.
        self.ok(unsafe { ffi::hbr_begin_tree(self.e(), rows.len() as u64, &mut root) })?;
        Some(self.issue(&root))
    }

    fn root_total(&self, gpair: Option<&[GradPair]>, rows: &[u32], seg: &Segment) -> Option<GradStats> {
        if rows.len() != seg.len() {
            return None;
        }
        let raw = self.raw(seg);
        let mut out = [0f64; 2];
        // SAFETY: writes two f64.
        let st = unsafe { ffi::hbr_root_total(self.e(), &raw, out.as_mut_ptr()) };
        match st {
            ffi::HBR_OK => Some(GradStats::new(out[0], out[1])),
            ffi::HBR_REFUSED => {
                // outside the exact domain: `sum_rows`'s row-order chain on the host
                let downloaded = match gpair {
                    Some(_) => None,
                    None => Some(self.device_gradients()?),
                };
                let pairs = gpair.or(downloaded.as_deref())?;
                let mut total = GradStats::default();
                for &r in rows {
                    total.add(GradStats::from_pair(*pairs.get(r as usize)?));
                }
                Some(total)
            }
            st => self.ok(st).map(|()| GradStats::default()),
        }
    }

    fn partition(&self, ghist: &GHistIndex, splits: Vec<RowSplit<'_>>) -> Option<Vec<Partitioned>> {
        if !self.fits(ghist) {
            return None;
        }
        // the tables' bytes live until the call returns
        let tables: Vec<Vec<u8>> = splits
            .iter()
            .map(|s| match s.rule {
                RowRule::Below(_) => Vec::new(),
                RowRule::Table(left) => left.iter().map(|&l| u8::from(l)).collect(),
            })
            .collect();
        let raw: Vec<ffi::hbr_row_split> = splits
            .iter()
            .zip(&tables)
            .map(|(s, table)| {
                let (below, n_table, table) = match s.rule {
                    RowRule::Below(limit) => (limit, 0, ptr::null()),
                    RowRule::Table(_) => (0, table.len() as u32, table.as_ptr()),
                };
                ffi::hbr_row_split {
                    seg: self.raw(&s.seg),
                    feature: s.feature,
                    below,
                    default_left: u32::from(s.default_left),
                    n_table,
                    table,
                }
            })
            .collect();
        let mut out = vec![ffi::hbr_partitioned::default(); raw.len()];
        // SAFETY: `raw.len()` splits in, as many partitions out.
        self.ok(unsafe { ffi::hbr_partition(self.e(), raw.as_ptr(), raw.len() as u64, out.as_mut_ptr()) })?;
        // the consumed segments are dropped with `splits`
        Some(
            out.iter()
                .map(|p| Partitioned {
                    left: self.issue(&p.left),
                    right: self.issue(&p.right),
                })
                .collect(),
        )
    }

    fn histograms(&self, ghist: &GHistIndex, gpair: Option<&[GradPair]>, nodes: &[&Segment]) -> Option<Vec<Histogram>> {
        if !self.fits(ghist) {
            return None;
        }
        let raw: Vec<ffi::hbr_segment> = nodes.iter().map(|s| self.raw(s)).collect();
        let mut flat = vec![GradStats::default(); nodes.len() * self.total_bins];
        // SAFETY: one histogram of total_bins (f64, f64) records per node.
        let st = unsafe {
            ffi::hbr_histograms(self.e(), raw.as_ptr(), raw.len() as u64, flat.as_mut_ptr().cast::<f64>())
        };
        match st {
            ffi::HBR_OK => Some(flat.chunks(self.total_bins.max(1)).map(<[GradStats]>::to_vec).collect()),
            ffi::HBR_REFUSED => {
                let downloaded = match gpair {
                    Some(_) => None,
                    None => Some(self.device_gradients()?),
                };
                let pairs = gpair.or(downloaded.as_deref())?;
                nodes.iter().map(|s| self.host_histogram(ghist, pairs, s)).collect()
            }
            st => self.ok(st).map(|()| Vec::new()),
        }
    }

    fn rows(&self, segs: &[&Segment]) -> Option<Vec<Vec<u32>>> {
        segs.iter().map(|s| self.segment_rows(s)).collect()
    }

    fn load_margins(&self, margins: &[f32]) -> Option<()> {
        if self.n_rows == 0 || margins.len() % self.n_rows != 0 {
            return None;
        }
        let outputs = u32::try_from(margins.len() / self.n_rows).ok()?;
        // SAFETY: n_rows * outputs f32, copied before return.
        self.ok(unsafe { ffi::hbr_load_margins(self.e(), margins.as_ptr(), margins.len() as u64, outputs) })
    }

    fn gradients(&self, loss: DeviceLoss, labels: &[f32], weights: Option<&[f32]>) -> Option<bool> {
        let raw = match loss {
            DeviceLoss::SquaredError { scale_pos_weight } => ffi::hbr_device_loss {
                kind: ffi::HBR_LOSS_SQUARED_ERROR,
                scale_pos_weight,
                min_hess: 0.0,
                max_input: 0.0,
                vector_rows: 0,
            },
            DeviceLoss::Logistic {
                scale_pos_weight,
                min_hess,
                split,
            } => {
                // the device restates the 8-lane kernel; a NEON (4-lane) host runs the rows itself
                if split.rows > 0 && split.lanes != DEVICE_VECTOR_LANES {
                    return None;
                }
                ffi::hbr_device_loss {
                    kind: ffi::HBR_LOSS_LOGISTIC,
                    scale_pos_weight,
                    min_hess,
                    max_input: split.max_input,
                    vector_rows: split.rows as u64,
                }
            }
        };
        if labels.len() != self.n_rows || weights.is_some_and(|w| w.len() != self.n_rows) {
            return None;
        }
        let mut finite: c_int = 0;
        let w = weights.map_or(ptr::null(), <[f32]>::as_ptr);
        // SAFETY: n_rows labels (and weights), read on the first call of a
        // margin run and kept until the next `load_margins`, which the trait
        // requires to stay unchanged meanwhile.
        self.ok(unsafe { ffi::hbr_gradients(self.e(), &raw, labels.as_ptr(), w, labels.len() as u64, &mut finite) })?;
        Some(finite != 0)
    }

    fn add_leaf_values(&self, leaves: Vec<(Segment, f32)>) -> Option<()> {
        let segs: Vec<ffi::hbr_segment> = leaves.iter().map(|(s, _)| self.raw(s)).collect();
        let values: Vec<f32> = leaves.iter().map(|&(_, v)| v).collect();
        // SAFETY: as many values as segments.
        self.ok(unsafe { ffi::hbr_add_leaf_values(self.e(), segs.as_ptr(), values.as_ptr(), segs.len() as u64) })
    }

    fn read_margins(&self, out: &mut [f32]) -> Option<()> {
        // SAFETY: `out.len()` f32.
        self.ok(unsafe { ffi::hbr_read_margins(self.e(), out.as_mut_ptr(), out.len() as u64) })
    }

    fn reserve_hists(&self, ghist: &GHistIndex, slots: usize) -> Option<bool> {
        if !self.fits(ghist) {
            return None;
        }
        let mut fits: c_int = 0;
        // SAFETY: writes one int.
        self.ok(unsafe { ffi::hbr_reserve_hists(self.e(), slots as u64, &mut fits) })?;
        Some(fits != 0)
    }

    fn build_resident(
        &self,
        ghist: &GHistIndex,
        _gpair: Option<&[GradPair]>,
        nodes: &[(&Segment, HistSlot)],
        siblings: &[(HistSlot, HistSlot)],
    ) -> Option<()> {
        if !self.fits(ghist) {
            return None;
        }
        let segs: Vec<ffi::hbr_segment> = nodes.iter().map(|(s, _)| self.raw(s)).collect();
        let slots: Vec<u32> = nodes.iter().map(|&(_, slot)| slot).collect();
        let parents: Vec<u32> = siblings.iter().map(|&(p, _)| p).collect();
        let built: Vec<u32> = siblings.iter().map(|&(_, b)| b).collect();
        // SAFETY: matching lengths as passed. A refusal (sums outside the
        // exact domain) leaves the slots as they were: `None` sends the
        // builder to its host path.
        self.ok(unsafe {
            ffi::hbr_build_resident(
                self.e(),
                segs.as_ptr(),
                slots.as_ptr(),
                segs.len() as u64,
                parents.as_ptr(),
                built.as_ptr(),
                parents.len() as u64,
            )
        })
    }

    fn scan_resident(&self, ghist: &GHistIndex, reg: &RegParams, requests: &[ScanRequest<'_>]) -> Option<Vec<NodeScan>> {
        if !self.fits(ghist) {
            return None;
        }
        // per request: the features and monotone directions as two arrays
        let features: Vec<Vec<u32>> = requests.iter().map(|r| r.features.iter().map(|&(f, _)| f).collect()).collect();
        let directions: Vec<Vec<i8>> = requests.iter().map(|r| r.features.iter().map(|&(_, d)| d).collect()).collect();
        let raw: Vec<ffi::hbr_scan_request> = requests
            .iter()
            .zip(features.iter().zip(&directions))
            .map(|(r, (f, d))| ffi::hbr_scan_request {
                slot: r.slot,
                has_fixed: 0,
                total_g: r.total.grad,
                total_h: r.total.hess,
                fixed_g: 0,
                fixed_h: 0,
                root_gain: r.root_gain,
                lower: r.lower,
                upper: r.upper,
                n_features: f.len() as u32,
                features: f.as_ptr(),
                directions: if d.iter().any(|&v| v != 0) { d.as_ptr() } else { ptr::null() },
            })
            .collect();
        let reg = ffi::hbr_reg_params {
            lambda: reg.lambda,
            alpha: reg.alpha,
            max_delta_step: reg.max_delta_step,
            min_child_weight: reg.min_child_weight,
        };
        let mut out = vec![ffi::hbr_node_scan::default(); raw.len()];
        // SAFETY: `raw.len()` requests in, as many results out; the feature
        // arrays outlive the call.
        self.ok(unsafe { ffi::hbr_scan_resident(self.e(), &reg, raw.as_ptr(), raw.len() as u64, out.as_mut_ptr()) })?;
        let pool_len = out
            .iter()
            .filter(|s| s.kind == ffi::HBR_SCAN_CATEGORICAL)
            .map(|s| s.cat_end as usize)
            .max()
            .unwrap_or(0);
        let mut pool = vec![0u32; pool_len];
        // SAFETY: the pool's length, as the scan reported it.
        self.ok(unsafe { ffi::hbr_scan_categories(self.e(), pool.as_mut_ptr(), pool_len as u64) })?;
        Some(
            out.iter()
                .map(|s| match s.kind {
                    ffi::HBR_SCAN_NUMERIC => NodeScan::Numeric {
                        feature: s.feature,
                        loss_chg: s.loss_chg,
                        backward: s.backward != 0,
                        offset: s.offset,
                        acc: GradStats::new(s.acc_g, s.acc_h),
                    },
                    ffi::HBR_SCAN_CATEGORICAL => NodeScan::Categorical {
                        feature: s.feature,
                        loss_chg: s.loss_chg,
                        default_left: s.default_left != 0,
                        left: GradStats::new(s.left_g, s.left_h),
                        right: GradStats::new(s.right_g, s.right_h),
                        categories: pool[s.cat_begin as usize..s.cat_end as usize].to_vec(),
                    },
                    // a near tie comes back only with HBR_GUARD_REPLAY (this module
                    // resolves them on the device): the builder replays the node from
                    // read_hist, which returns the CPU builder's own sums
                    ffi::HBR_SCAN_REPLAY => NodeScan::Replay(match s.fallback {
                        ffi::HBR_FALLBACK_CATEGORICAL_ORDER => ScanFallback::CategoricalOrder,
                        ffi::HBR_FALLBACK_CATEGORICAL_SCORE => ScanFallback::CategoricalScore,
                        _ => ScanFallback::NumericScore,
                    }),
                    _ => NodeScan::Empty,
                })
                .collect(),
        )
    }

    fn read_hist(&self, slot: HistSlot) -> Option<Histogram> {
        let mut out = vec![GradStats::default(); self.total_bins];
        // SAFETY: total_bins (f64, f64) records.
        self.ok(unsafe { ffi::hbr_read_hist(self.e(), slot, out.as_mut_ptr().cast::<f64>()) })?;
        Some(out)
    }
}

