//! Batch prediction on the MI355X: [`BoostedModel::to_rocm`] uploads a
//! model's forest once, [`RocmModel`] walks it over `DMatrix` rows on the GPU
//! (the counterpart of `GpuModel`, src/backend/cuda/predict.rs:358-480).
//! Margins are the CPU's bit for bit: each row starts from the model's
//! initial margins (the base scores, or the matrix's base_margin) and adds
//! every tree's `weight * leaf` in tree order, in f32; categorical splits
//! and DART weights included. The objective's transform and model-shrinkage
//! prediction run on the CPU, as for CUDA (`plan_margins`,
//! src/backend/shared.rs:218-239).

use super::{check, ffi};
use crate::backend::shared::{MarginPlan, ensure_forest_model, plan_margins};
use crate::data::DMatrix;
use crate::error::{HessboostError, Result};
use crate::model::{BoostedModel, Iterations, Predictions};
use std::ops::Range;
use std::os::raw::c_int;
use std::ptr::{self, NonNull};
use std::sync::{Arc, Mutex};

/// Rows per library call: the dense copy of a CSR block and the device
/// buffers of one call stay bounded (at most 2^22 rows, and at most 2^28
/// f32 cells of features plus outputs).
const BLOCK_CELLS: usize = 1 << 28;
const BLOCK_ROWS: usize = 1 << 22;

/// One uploaded forest (`hbr_forest`).
struct Forest(NonNull<ffi::hbr_forest>);

// SAFETY: the library serializes calls on a forest behind its own mutex.
unsafe impl Send for Forest {}
// SAFETY: as above.
unsafe impl Sync for Forest {}

impl Drop for Forest {
    fn drop(&mut self) {
        // SAFETY: uploaded by `hbr_forest_upload`, freed once.
        unsafe { ffi::hbr_forest_free(self.0.as_ptr()) }
    }
}

/// A model resident on one ROCm device, built with
/// [`BoostedModel::to_rocm`]. Calls may run concurrently.
pub struct RocmModel {
    model: Arc<BoostedModel>,
    ordinal: usize,
    /// Forests by tree range: the whole model, uploaded by `to_rocm`, then
    /// any iteration range a prediction asks for, uploaded once.
    forests: Mutex<Vec<(Range<usize>, Arc<Forest>)>>,
}

impl std::fmt::Debug for RocmModel {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        f.debug_struct("RocmModel")
            .field("model", &self.model)
            .field("ordinal", &self.ordinal)
            .finish_non_exhaustive()
    }
}

/// The node arrays of trees `trees` in the library's forest layout
/// (`hbr_forest_desc`: the reference's `Node` fields, src/tree/regtree.rs:
/// 38-66, one array per field; categorical nodes' ranges into one pool).
fn upload(model: &BoostedModel, trees: Range<usize>, ordinal: usize) -> Result<Forest> {
    let mut tree_offset = vec![0u64];
    let (mut split_feature, mut split_cond, mut default_left) = (Vec::new(), Vec::new(), Vec::new());
    let (mut left, mut right, mut leaf_value) = (Vec::new(), Vec::new(), Vec::new());
    let (mut is_categorical, mut cat_begin, mut cat_end) = (Vec::new(), Vec::new(), Vec::new());
    let (mut categories, mut tree_weight, mut tree_output) = (Vec::new(), Vec::new(), Vec::new());
    for t in trees {
        let tree = &model.trees()[t];
        if tree.is_vector_leaf() {
            return Err(HessboostError::incompatible_model(
                "model",
                "rocm prediction holds scalar leaves only; vector-leaf models predict on the CPU",
            ));
        }
        let pool = u32::try_from(categories.len())
            .map_err(|_| HessboostError::invalid_data("model", "rocm: category pool beyond 2^32"))?;
        for node in tree.nodes() {
            split_feature.push(node.split_feature);
            split_cond.push(node.split_cond);
            default_left.push(u8::from(node.default_left));
            left.push(node.left);
            right.push(node.right);
            leaf_value.push(node.leaf_value);
            is_categorical.push(u8::from(node.is_categorical));
            cat_begin.push(pool + node.cat_begin);
            cat_end.push(pool + node.cat_end);
        }
        categories.extend_from_slice(tree.categories());
        tree_offset.push(split_feature.len() as u64);
        tree_weight.push(model.tree_weight(t));
        tree_output.push(
            u32::try_from(model.tree_output(t))
                .map_err(|_| HessboostError::invalid_data("model", "rocm: output index beyond 2^32"))?,
        );
    }
    let n_outputs = u32::try_from(model.n_outputs())
        .map_err(|_| HessboostError::invalid_data("model", "rocm: more than 2^32 outputs"))?;
    let base_score = model.base_scores();
    let desc = ffi::hbr_forest_desc {
        n_trees: tree_weight.len() as u64,
        tree_offset: tree_offset.as_ptr(),
        split_feature: split_feature.as_ptr(),
        split_cond: split_cond.as_ptr(),
        default_left: default_left.as_ptr(),
        left: left.as_ptr(),
        right: right.as_ptr(),
        leaf_value: leaf_value.as_ptr(),
        tree_weight: tree_weight.as_ptr(),
        tree_output: tree_output.as_ptr(),
        n_outputs,
        pad: 0,
        base_score: base_score.as_ptr(),
        is_categorical: is_categorical.as_ptr(),
        cat_begin: cat_begin.as_ptr(),
        cat_end: cat_end.as_ptr(),
        categories: if categories.is_empty() { ptr::null() } else { categories.as_ptr() },
        n_categories: categories.len() as u64,
    };
    let ordinal = c_int::try_from(ordinal)
        .map_err(|_| HessboostError::invalid_param("device", "rocm ordinal out of range"))?;
    let mut forest = ptr::null_mut();
    // SAFETY: every array of `desc` outlives the call; the library copies
    // the forest to the device and keeps nothing of the host's.
    check(unsafe { ffi::hbr_forest_upload(ordinal, &desc, &mut forest) })?;
    NonNull::new(forest).map(Forest).ok_or_else(|| HessboostError::gpu("rocm: no forest"))
}

impl RocmModel {
    /// The source model, including its CPU objective transform.
    #[must_use]
    pub fn model(&self) -> &BoostedModel {
        &self.model
    }

    /// The ROCm device ordinal this model resides on.
    #[must_use]
    pub fn ordinal(&self) -> usize {
        self.ordinal
    }

    fn forest(&self, trees: Range<usize>) -> Result<Arc<Forest>> {
        let mut forests = self.forests.lock().unwrap_or_else(std::sync::PoisonError::into_inner);
        if let Some((_, f)) = forests.iter().find(|(r, _)| *r == trees) {
            return Ok(Arc::clone(f));
        }
        let f = Arc::new(upload(&self.model, trees.clone(), self.ordinal)?);
        forests.push((trees, Arc::clone(&f)));
        Ok(f)
    }

    /// Raw margins, bit-identical to [`BoostedModel::predict_margin`].
    pub fn predict_margin(&self, data: &DMatrix, iterations: impl Into<Iterations>) -> Result<Predictions> {
        let (trees, mut margins) = match plan_margins(&self.model, data, iterations.into())? {
            MarginPlan::Done(margins) => return Ok(margins),
            MarginPlan::Walk { trees, margins } => (trees, margins),
        };
        let forest = self.forest(trees)?;
        let (n, n_cols, k) = (data.n_rows(), data.n_cols(), self.model.n_outputs());
        let missing = data.missing();
        let block = (BLOCK_CELLS / (n_cols + k).max(1)).clamp(1, BLOCK_ROWS);
        let mut rows = Vec::new();
        let mut out = Vec::new();
        for r0 in (0..n).step_by(block) {
            let m = block.min(n - r0);
            // the block's rows, row-major f32; absent cells hold the sentinel
            let x: &[f32] = match data.dense_rows() {
                Some(dense) => match dense.contiguous() {
                    Some(all) => &all[r0 * n_cols..(r0 + m) * n_cols],
                    None => {
                        rows.clear();
                        (r0..r0 + m).for_each(|r| rows.extend_from_slice(dense.row(r)));
                        &rows
                    }
                },
                None => {
                    let csr = data
                        .csr_rows()
                        .ok_or_else(|| HessboostError::invalid_data("data", "rocm: a matrix without values"))?;
                    rows.clear();
                    rows.resize(m * n_cols, missing);
                    for r in 0..m {
                        let (cols, values) = csr.row(r0 + r);
                        for (&c, &v) in cols.iter().zip(values) {
                            rows[r * n_cols + c as usize] = v;
                        }
                    }
                    &rows
                }
            };
            out.resize(m * k, 0.0);
            let init = &margins[r0 * k..(r0 + m) * k];
            // SAFETY: m rows of n_cols f32, m * k starting margins and as
            // many outputs, all host memory that outlives the call.
            check(unsafe {
                ffi::hbr_predict_margin_from(
                    forest.0.as_ptr(),
                    x.as_ptr(),
                    m as u64,
                    n_cols as u64,
                    missing,
                    init.as_ptr(),
                    out.as_mut_ptr(),
                )
            })?;
            margins[r0 * k..(r0 + m) * k].copy_from_slice(&out);
        }
        Ok(Predictions::new(margins, n, k))
    }

    /// Predictions with the CPU's exact objective transform.
    pub fn predict(&self, data: &DMatrix, iterations: impl Into<Iterations>) -> Result<Predictions> {
        Ok(self.model.transform_margins(self.predict_margin(data, iterations)?))
    }

    /// Predicted classes, as for [`BoostedModel::predict_class`].
    pub fn predict_class(&self, data: &DMatrix, iterations: impl Into<Iterations>) -> Result<Predictions<u32>> {
        Ok(self.model.classes(&self.predict(data, iterations)?))
    }
}

impl BoostedModel {
    /// Upload the forest once to ROCm device `ordinal` (an MI355X, gfx950),
    /// beside [`BoostedModel::to_cuda`] (src/model/mod.rs:1046-1056).
    /// Refuses `gblinear`, per-leaf linear and vector-leaf models.
    pub fn to_rocm(&self, ordinal: usize) -> Result<RocmModel> {
        ensure_forest_model(self)?;
        let model = Arc::new(self.clone());
        let all = 0..model.num_trees();
        let forest = Arc::new(upload(&model, all.clone(), ordinal)?);
        Ok(RocmModel {
            model,
            ordinal,
            forests: Mutex::new(vec![(all, forest)]),
        })
    }
}
