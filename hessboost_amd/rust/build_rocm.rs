// Linking the MI355X backend into hessboost: the `rocm` feature's part of
// the crate's `build.rs`. hessboost declares the feature with no
// dependencies (`rocm = []` under [features] in Cargo.toml) and calls
// `link_rocm()` first thing in `main`.
//
// HBROCM_LIB_DIR names the directory holding `libhbrocm.so` and its code
// object `hbrocm_gfx950.hsaco` (built by `make -C hessboost_amd/csrc`,
// output in `hessboost_amd/lib/`). The rpath lets the test binaries and
// examples find the library without LD_LIBRARY_PATH; the library locates
// its code object beside itself at run time.

fn link_rocm() {
    if std::env::var_os("CARGO_FEATURE_ROCM").is_none() {
        return;
    }
    println!("cargo:rerun-if-env-changed=HBROCM_LIB_DIR");
    let dir = std::env::var("HBROCM_LIB_DIR")
        .expect("the rocm feature needs HBROCM_LIB_DIR: the directory of libhbrocm.so");
    let lib = std::path::Path::new(&dir).join("libhbrocm.so");
    assert!(lib.is_file(), "{} is missing: build it with `make -C hessboost_amd/csrc`", lib.display());
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=hbrocm");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
}
