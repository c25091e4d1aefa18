// Links libmri_qmatmul.so (built for gfx950 by mini-rust-inference_amd/csrc)
// and the HIP runtime it needs.  MRI_LIB_DIR names the directory of the
// library; by default it is the package directory two levels up, where the
// build puts it.  ROCM_PATH (default /opt/rocm) locates libamdhip64.so.
use std::env;
use std::path::PathBuf;

fn main() {
    let lib_dir = match env::var("MRI_LIB_DIR") {
        Ok(d) => PathBuf::from(d),
        Err(_) => {
            let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
            manifest.join("..").join("..")
        }
    };
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={}", lib_dir.display());
    println!("cargo:rustc-link-search=native={}/lib", rocm);
    println!("cargo:rustc-link-lib=dylib=mri_qmatmul");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    // the library is found at run time without LD_LIBRARY_PATH
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", lib_dir.display());
    println!("cargo:rerun-if-env-changed=MRI_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    println!("cargo:rerun-if-changed=build.rs");
}
