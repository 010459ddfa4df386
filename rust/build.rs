// build.rs for the RustLLM crate on the gfx950 library: links
// librustllm_hip.so (built with `python -m rustllm_amd.build`, hipcc for
// gfx950) in place of the `metal` crate, which leaves Cargo.toml.
fn main() {
    let dir = std::env::var("RUSTLLM_HIP_LIB_DIR")
        .expect("set RUSTLLM_HIP_LIB_DIR to the directory holding librustllm_hip.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=rustllm_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    println!("cargo:rerun-if-env-changed=RUSTLLM_HIP_LIB_DIR");
}
