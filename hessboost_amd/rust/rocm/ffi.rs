//! Declarations of the MI355X backend's C ABI (`include/hessboost_rocm.h`),
//! one for one: the handles, the argument records and every entry point. A
//! hessboost build with the `rocm` feature links `libhbrocm.so` (see
//! `build.rs` beside this file); its code object `hbrocm_gfx950.hsaco` must
//! sit in the library's directory.
//!
//! Every call returns a status: `HBR_OK`; `HBR_REFUSED` (the device does not
//! run this call for these inputs and changed nothing: the traits' `None`);
//! `HBR_DEVICE_ERROR` (a HIP error: the handle refuses every later call, the
//! CUDA backend's sticky `failed` flag, src/backend/cuda/mod.rs:1806-1826);
//! `HBR_INVALID` (malformed arguments). `hbr_last_error` gives the calling
//! thread's message. Pointers are host pointers unless a name says device.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

pub const HBR_OK: c_int = 0;
pub const HBR_REFUSED: c_int = 1;
pub const HBR_DEVICE_ERROR: c_int = 2;
pub const HBR_INVALID: c_int = 3;

pub const HBR_SUMS_EXACT: c_int = 0;
pub const HBR_SUMS_FIXED_POINT: c_int = 1;

pub const HBR_LOSS_SQUARED_ERROR: u32 = 0;
pub const HBR_LOSS_LOGISTIC: u32 = 1;
pub const HBR_LOSS_SOFTMAX: u32 = 2;

pub const HBR_SCAN_EMPTY: u32 = 0;
pub const HBR_SCAN_REPLAY: u32 = 1;
pub const HBR_SCAN_NUMERIC: u32 = 2;
pub const HBR_SCAN_CATEGORICAL: u32 = 3;
pub const HBR_FALLBACK_NUMERIC_SCORE: u32 = 1;
pub const HBR_FALLBACK_CATEGORICAL_ORDER: u32 = 2;
pub const HBR_FALLBACK_CATEGORICAL_SCORE: u32 = 3;
pub const HBR_FALLBACK_NEAR_TIE: u32 = 4;
pub const HBR_GUARD_OFF: c_int = 0;
pub const HBR_GUARD_REPLAY: c_int = 1;
pub const HBR_GUARD_RESOLVE: c_int = 2;

pub const HBR_OBJ_SQUARED_ERROR: i32 = 0;
pub const HBR_OBJ_LOGISTIC: i32 = 1;
pub const HBR_OBJ_SOFTMAX: i32 = 2;
pub const HBR_OBJ_LOGITRAW: i32 = 3;
pub const HBR_GROW_DEPTHWISE: i32 = 0;
pub const HBR_GROW_LOSSGUIDE: i32 = 1;

pub const HBR_TRANSFORM_SIGMOID: c_int = 1;
pub const HBR_TRANSFORM_SOFTMAX: c_int = 2;
pub const HBR_TRANSFORM_CLASS_INDEX: c_int = 3;

// Opaque handles.
#[repr(C)]
pub struct hbr_cuts {
    _private: [u8; 0],
}
#[repr(C)]
pub struct hbr_index {
    _private: [u8; 0],
}
#[repr(C)]
pub struct hbr_engine {
    _private: [u8; 0],
}
#[repr(C)]
pub struct hbr_trainer {
    _private: [u8; 0],
}
#[repr(C)]
pub struct hbr_forest {
    _private: [u8; 0],
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct hbr_index_desc {
    pub n_rows: u64,
    pub n_cols: u64,
    pub feature_offset: *const u32,
    pub cut_values: *const f32,
    pub row_ptr: *const u64,
    pub row_bins: *const c_void,
    pub row_bin_width: u32,
    pub dense: u32,
    pub col_bins: *const c_void,
    pub col_bin_width: u32,
    pub pad: u32,
    pub missing: *const u64,
    pub is_categorical: *const u8,
}

#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct hbr_index_info {
    pub dense: u32,
    pub dense_u8: u32,
    pub has_cols: u32,
    pub has_missing: u32,
    pub stride: u32,
    pub pad: u32,
    pub entries: u64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct hbr_segment {
    pub offset: u64,
    pub len: u64,
    pub buffer: u32,
    pub contiguous: u32,
    pub tree: u64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct hbr_row_split {
    pub seg: hbr_segment,
    pub feature: u32,
    pub below: u32,
    pub default_left: u32,
    pub n_table: u32,
    pub table: *const u8,
}

#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct hbr_partitioned {
    pub left: hbr_segment,
    pub right: hbr_segment,
}

#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct hbr_device_loss {
    pub kind: u32,
    pub scale_pos_weight: f32,
    pub min_hess: f32,
    pub max_input: f32,
    pub vector_rows: u64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct hbr_reg_params {
    pub lambda: f64,
    pub alpha: f64,
    pub max_delta_step: f64,
    pub min_child_weight: f64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct hbr_scan_request {
    pub slot: u32,
    pub has_fixed: u32,
    pub total_g: f64,
    pub total_h: f64,
    pub fixed_g: i64,
    pub fixed_h: i64,
    pub root_gain: f32,
    pub lower: f32,
    pub upper: f32,
    pub n_features: u32,
    pub features: *const u32,
    pub directions: *const i8,
}

#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct hbr_node_scan {
    pub kind: u32,
    pub feature: u32,
    pub loss_chg: f32,
    pub backward: u32,
    pub offset: u32,
    pub loss_err: f32,
    pub acc_g: f64,
    pub acc_h: f64,
    pub left_g: f64,
    pub left_h: f64,
    pub right_g: f64,
    pub right_h: f64,
    pub fixed_left_g: i64,
    pub fixed_left_h: i64,
    pub fixed_right_g: i64,
    pub fixed_right_h: i64,
    pub default_left: u32,
    pub fallback: u32,
    pub cat_begin: u32,
    pub cat_end: u32,
}

#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct hbr_engine_counters {
    pub hist_nodes: u64,
    pub hist_rows: u64,
    pub hist_bytes: u64,
    pub partition_rows: u64,
    pub trees: u64,
    pub near_ties: u64,
    pub near_ties_resolved: u64,
    pub row_orders: u64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct hbr_train_params {
    pub eta: f64,
    pub gamma: f64,
    pub lambda: f64,
    pub alpha: f64,
    pub min_child_weight: f64,
    pub max_delta_step: f64,
    pub max_depth: i64,
    pub max_leaves: i64,
    pub grow_policy: i32,
    pub objective: i32,
    pub num_class: i32,
    pub scale_pos_weight: f32,
    pub monotone: *const i8,
    pub n_monotone: u64,
    pub base_score: f32,
    pub has_base_score: i32,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct hbr_forest_desc {
    pub n_trees: u64,
    pub tree_offset: *const u64,
    pub split_feature: *const u32,
    pub split_cond: *const f32,
    pub default_left: *const u8,
    pub left: *const i32,
    pub right: *const i32,
    pub leaf_value: *const f32,
    pub tree_weight: *const f32,
    pub tree_output: *const u32,
    pub n_outputs: u32,
    pub pad: u32,
    pub base_score: *const f32,
    pub is_categorical: *const u8,
    pub cat_begin: *const u32,
    pub cat_end: *const u32,
    pub categories: *const u32,
    pub n_categories: u64,
}

extern "C" {
    pub fn hbr_last_error(buf: *mut c_char, len: usize) -> usize;
    pub fn hbr_device_count(count: *mut c_int) -> c_int;
    pub fn hbr_device_name(ordinal: c_int, buf: *mut c_char, len: usize) -> c_int;
    pub fn hbr_cuts_from_dense(x: *const f32, n_rows: u64, n_cols: u64, max_bin: u32, weights: *const f32,
                               missing: f32, out: *mut *mut hbr_cuts) -> c_int;
    pub fn hbr_cuts_from_csr(row_ptr: *const u64, col: *const u32, val: *const f32, n_rows: u64, n_cols: u64,
                             max_bin: u32, weights: *const f32, out: *mut *mut hbr_cuts) -> c_int;
    pub fn hbr_cuts_from_dense_typed(x: *const f32, n_rows: u64, n_cols: u64, max_bin: u32,
                                     weights: *const f32, missing: f32, categorical: *const u8,
                                     out: *mut *mut hbr_cuts) -> c_int;
    pub fn hbr_cuts_from_csr_typed(row_ptr: *const u64, col: *const u32, val: *const f32, n_rows: u64,
                                   n_cols: u64, max_bin: u32, weights: *const f32, categorical: *const u8,
                                   out: *mut *mut hbr_cuts) -> c_int;
    pub fn hbr_cuts_categorical(c: *const hbr_cuts, out: *mut u8) -> c_int;
    pub fn hbr_cuts_from_values(feature_offset: *const u32, cut_values: *const f32, n_cols: u64,
                                out: *mut *mut hbr_cuts) -> c_int;
    pub fn hbr_cuts_info(c: *const hbr_cuts, n_cols: *mut u64, total_bins: *mut u64) -> c_int;
    pub fn hbr_cuts_copy(c: *const hbr_cuts, feature_offset: *mut u32, cut_values: *mut f32) -> c_int;
    pub fn hbr_cuts_free(c: *mut hbr_cuts);
    pub fn hbr_index_from_dense(x: *const f32, n_rows: u64, n_cols: u64, missing: f32, cuts: *const hbr_cuts,
                                out: *mut *mut hbr_index) -> c_int;
    pub fn hbr_index_from_csr(row_ptr: *const u64, col: *const u32, val: *const f32, n_rows: u64,
                              n_cols: u64, cuts: *const hbr_cuts, out: *mut *mut hbr_index) -> c_int;
    pub fn hbr_index_free(ix: *mut hbr_index);
    pub fn hbr_index_describe(ix: *const hbr_index, out: *mut hbr_index_desc) -> c_int;
    pub fn hbr_engine_open(ordinal: c_int, index: *const hbr_index_desc, out: *mut *mut hbr_engine) -> c_int;
    pub fn hbr_engine_close(e: *mut hbr_engine);
    pub fn hbr_engine_open_dense(ordinal: c_int, x: *const f32, n_rows: u64, n_cols: u64, missing: f32,
                                 cuts: *const hbr_cuts, x_on_device: c_int, out: *mut *mut hbr_engine) -> c_int;
    pub fn hbr_engine_index_info(e: *mut hbr_engine, out: *mut hbr_index_info) -> c_int;
    pub fn hbr_engine_index_read(e: *mut hbr_engine, rows8: *mut u8, cols8: *mut u8, missing: *mut u64,
                                 row_ptr: *mut u64, gbins: *mut u32) -> c_int;
    pub fn hbr_engine_set_sums(e: *mut hbr_engine, mode: c_int) -> c_int;
    pub fn hbr_prepare(e: *mut hbr_engine, gpair: *const f32, n: u64) -> c_int;
    pub fn hbr_build(e: *mut hbr_engine, rows: *const u32, m: u64, out: *mut f64) -> c_int;
    pub fn hbr_build_device_noalloc(e: *mut hbr_engine, rows: *const u32, m: u64, out: *mut f64) -> c_int;
    pub fn hbr_begin_tree(e: *mut hbr_engine, n_rows: u64, root: *mut hbr_segment) -> c_int;
    pub fn hbr_root_total(e: *mut hbr_engine, seg: *const hbr_segment, out: *mut f64) -> c_int;
    pub fn hbr_partition(e: *mut hbr_engine, splits: *const hbr_row_split, n: u64, out: *mut hbr_partitioned) -> c_int;
    pub fn hbr_histograms(e: *mut hbr_engine, segs: *const hbr_segment, n: u64, out: *mut f64) -> c_int;
    pub fn hbr_rows(e: *mut hbr_engine, seg: *const hbr_segment, out: *mut u32) -> c_int;
    pub fn hbr_load_margins(e: *mut hbr_engine, margins: *const f32, n: u64, n_outputs: u32) -> c_int;
    pub fn hbr_gradients(e: *mut hbr_engine, loss: *const hbr_device_loss, labels: *const f32,
                         weights: *const f32, n: u64, all_finite: *mut c_int) -> c_int;
    pub fn hbr_read_gradients(e: *mut hbr_engine, out: *mut f32, n: u64) -> c_int;
    pub fn hbr_add_leaf_values(e: *mut hbr_engine, segs: *const hbr_segment, values: *const f32, n: u64) -> c_int;
    pub fn hbr_read_margins(e: *mut hbr_engine, out: *mut f32, n: u64) -> c_int;
    pub fn hbr_engine_add_eval(e: *mut hbr_engine, x: *const f32, n_rows: u64, n_cols: u64, missing: f32,
                               init_margins: *const f32, n_outputs: u32, index: *mut u32) -> c_int;
    pub fn hbr_engine_eval_add_tree(e: *mut hbr_engine, split_feature: *const u32, split_cond: *const f32,
                                    default_left: *const u8, left: *const i32, right: *const i32,
                                    leaf_value: *const f32, n_nodes: u64, output: u32) -> c_int;
    pub fn hbr_engine_eval_add_tree_categorical(e: *mut hbr_engine, split_feature: *const u32,
                                                split_cond: *const f32, default_left: *const u8, left: *const i32,
                                                right: *const i32, leaf_value: *const f32,
                                                is_categorical: *const u8, cat_begin: *const u32,
                                                cat_end: *const u32, categories: *const u32, n_categories: u64,
                                                n_nodes: u64, output: u32) -> c_int;
    pub fn hbr_engine_eval_margins(e: *mut hbr_engine, index: u32, out: *mut f32) -> c_int;
    pub fn hbr_reserve_hists(e: *mut hbr_engine, slots: u64, fits: *mut c_int) -> c_int;
    pub fn hbr_build_resident(e: *mut hbr_engine, segs: *const hbr_segment, slots: *const u32, n: u64,
                              sibling_parent: *const u32, sibling_built: *const u32, n_siblings: u64) -> c_int;
    pub fn hbr_root_total_fixed(e: *mut hbr_engine, seg: *const hbr_segment, out: *mut f64, fixed: *mut i64) -> c_int;
    pub fn hbr_scan_resident(e: *mut hbr_engine, reg: *const hbr_reg_params,
                             requests: *const hbr_scan_request, n: u64, out: *mut hbr_node_scan) -> c_int;
    pub fn hbr_scan_categories(e: *mut hbr_engine, out: *mut u32, n: u64) -> c_int;
    pub fn hbr_read_hist(e: *mut hbr_engine, slot: u32, out: *mut f64) -> c_int;
    pub fn hbr_engine_set_guard(e: *mut hbr_engine, mode: c_int, gamma: f64) -> c_int;
    pub fn hbr_node_gain(reg: *const hbr_reg_params, g: f64, h: f64, lower: f64, upper: f64, out: *mut f32) -> c_int;
    pub fn hbr_leaf_weight(reg: *const hbr_reg_params, g: f64, h: f64, lower: f64, upper: f64, out: *mut f32)
                           -> c_int;
    pub fn hbr_engine_counters_read(e: *mut hbr_engine, out: *mut hbr_engine_counters) -> c_int;
    pub fn hbr_set_profiling(e: *mut hbr_engine, on: c_int, kernel_prefix: *const c_char) -> c_int;
    pub fn hbr_kernel_stats(e: *mut hbr_engine, buf: *mut c_char, len: usize) -> c_int;
    pub fn hbr_trainer_create(e: *mut hbr_engine, p: *const hbr_train_params, labels: *const f32,
                              weights: *const f32, n_rows: u64, out: *mut *mut hbr_trainer) -> c_int;
    pub fn hbr_trainer_boost(t: *mut hbr_trainer, rounds: u64) -> c_int;
    pub fn hbr_trainer_num_trees(t: *mut hbr_trainer, n: *mut u64) -> c_int;
    pub fn hbr_trainer_num_outputs(t: *mut hbr_trainer, k: *mut u32) -> c_int;
    pub fn hbr_trainer_base_score(t: *mut hbr_trainer, out: *mut f32) -> c_int;
    pub fn hbr_trainer_tree_size(t: *mut hbr_trainer, tree: u64, n_nodes: *mut u64) -> c_int;
    pub fn hbr_trainer_tree(t: *mut hbr_trainer, tree: u64, split_feature: *mut u32, split_cond: *mut f32,
                            default_left: *mut u8, left: *mut i32, right: *mut i32, leaf_value: *mut f32,
                            sum_hess: *mut f32, split_gain: *mut f32, split_bin: *mut i64) -> c_int;
    pub fn hbr_trainer_tree_categories(t: *mut hbr_trainer, tree: u64, is_categorical: *mut u8,
                                       cat_begin: *mut u32, cat_end: *mut u32, categories: *mut u32,
                                       n_categories: *mut u64) -> c_int;
    pub fn hbr_trainer_margins(t: *mut hbr_trainer, out: *mut f32) -> c_int;
    pub fn hbr_trainer_add_eval(t: *mut hbr_trainer, x: *const f32, n_rows: u64, n_cols: u64, missing: f32,
                                base_margin: *const f32, index: *mut u32) -> c_int;
    pub fn hbr_trainer_eval_margins(t: *mut hbr_trainer, index: u32, out: *mut f32) -> c_int;
    pub fn hbr_trainer_free(t: *mut hbr_trainer);
    pub fn hbr_forest_upload(ordinal: c_int, fd: *const hbr_forest_desc, out: *mut *mut hbr_forest) -> c_int;
    pub fn hbr_forest_free(f: *mut hbr_forest);
    pub fn hbr_predict_margin(f: *mut hbr_forest, x: *const f32, n_rows: u64, n_cols: u64, missing: f32,
                              out: *mut f32) -> c_int;
    pub fn hbr_predict_margin_from(f: *mut hbr_forest, x: *const f32, n_rows: u64, n_cols: u64, missing: f32,
                                   init_margins: *const f32, out: *mut f32) -> c_int;
    pub fn hbr_predict_margin_device(f: *mut hbr_forest, x: *const f32, n_rows: u64, n_cols: u64,
                                     missing: f32, out: *mut f32, leaf_out: *mut i32) -> c_int;
    pub fn hbr_predict_leaf(f: *mut hbr_forest, x: *const f32, n_rows: u64, n_cols: u64, missing: f32,
                            out: *mut i32) -> c_int;
    pub fn hbr_forest_set_profiling(f: *mut hbr_forest, on: c_int, kernel_prefix: *const c_char) -> c_int;
    pub fn hbr_forest_kernel_stats(f: *mut hbr_forest, buf: *mut c_char, len: usize) -> c_int;
    pub fn hbr_pred_transform(kind: c_int, values: *mut f32, n_rows: u64, n_outputs: u32) -> c_int;
    pub fn hbr_device_alloc(ordinal: c_int, bytes: u64, out: *mut *mut c_void) -> c_int;
    pub fn hbr_device_free(ordinal: c_int, p: *mut c_void) -> c_int;
    pub fn hbr_device_upload(ordinal: c_int, dst: *mut c_void, src: *const c_void, bytes: u64) -> c_int;
    pub fn hbr_device_download(ordinal: c_int, dst: *mut c_void, src: *const c_void, bytes: u64) -> c_int;
    pub fn hbr_device_copy(ordinal: c_int, dst: *mut c_void, src: *const c_void, bytes: u64) -> c_int;
}
