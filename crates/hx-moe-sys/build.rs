// Link search path for libhxmoe.so: $HX_MOE_LIB_DIR, else the helexa_amd/
// directory of this repository (where `python -m helexa_amd.build` puts it).
fn main() {
    let dir = std::env::var("HX_MOE_LIB_DIR").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").unwrap();
        format!("{here}/../../helexa_amd")
    });
    println!("cargo:rerun-if-env-changed=HX_MOE_LIB_DIR");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=hxmoe");
}
