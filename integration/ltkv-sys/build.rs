// Links libltkv.so: LTKV_LIB_DIR names the directory holding it (the
// langtrain_studio_amd/ package directory after its build).
fn main() {
    if let Ok(dir) = std::env::var("LTKV_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    println!("cargo:rustc-link-lib=dylib=ltkv");
    println!("cargo:rerun-if-env-changed=LTKV_LIB_DIR");
}
