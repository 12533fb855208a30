// Links libcodon_hip.so.  CODON_HIP_LIB_DIR names the directory that holds
// it (codon-infer_amd/codon_hip after `python codon-infer_amd/build.py`);
// the directory is also written into the binary's run path.
fn main() {
    println!("cargo:rerun-if-env-changed=CODON_HIP_LIB_DIR");
    if let Ok(dir) = std::env::var("CODON_HIP_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    println!("cargo:rustc-link-lib=dylib=codon_hip");
}
