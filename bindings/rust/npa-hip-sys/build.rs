//! Links libnpa_hip.so. NPA_HIP_DIR names the directory that holds it (the repository's
//! burn_automata_amd/ after `python -m burn_automata_amd.build`); the HIP runtime it depends on is
//! found through the usual loader path (/opt/rocm/lib).
fn main() {
    println!("cargo:rerun-if-env-changed=NPA_HIP_DIR");
    if let Some(dir) = std::env::var_os("NPA_HIP_DIR") {
        println!("cargo:rustc-link-search=native={}", dir.to_string_lossy());
    }
    println!("cargo:rustc-link-search=native=/opt/rocm/lib");
    println!("cargo:rustc-link-lib=dylib=npa_hip");
}
