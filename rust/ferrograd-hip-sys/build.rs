// Links libferrograd_amd.so. FERROGRAD_AMD_LIB_DIR names the directory that
// holds it (the package directory ferrograd_amd/ after
// `python -c "import __graft_entry__ as g; g.build()"`); the default is the
// in-tree build two directories up. Not built in this repository (no cargo).
fn main() {
    let dir = std::env::var("FERROGRAD_AMD_LIB_DIR").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").expect("cargo sets CARGO_MANIFEST_DIR");
        format!("{here}/../../ferrograd_amd")
    });
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=ferrograd_amd");
    // The library finds its kernel code-object cache next to itself
    // (or in FG_KERNEL_CACHE); at run time the loader must find it too.
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    println!("cargo:rerun-if-env-changed=FERROGRAD_AMD_LIB_DIR");
}
