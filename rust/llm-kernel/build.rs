//! Links libllmk_sampler.so when the `hip-sampler` feature is on.  The
//! library's directory comes from LLMK_LIB_DIR (the directory `make -C
//! llm-rs_amd` writes it to); the HIP runtime it needs is found through the
//! library's own dependencies at load time.
fn main() {
    println!("cargo:rerun-if-env-changed=LLMK_LIB_DIR");
    if std::env::var_os("CARGO_FEATURE_HIP_SAMPLER").is_none() {
        return;
    }
    let dir = std::env::var("LLMK_LIB_DIR")
        .expect("the hip-sampler feature needs LLMK_LIB_DIR = the directory of libllmk_sampler.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=llmk_sampler");
    // the library is loaded from the same directory at run time
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
}
