//! Links liblightx2v_hip.so, built by `make -C lightx2v-rs_amd` (hipcc
//! --offload-arch=gfx950).  LIGHTX2V_HIP_LIB_DIR names the directory that
//! holds it (lightx2v-rs_amd/lightx2v_hip/ in the build tree).
fn main() {
    println!("cargo:rerun-if-env-changed=LIGHTX2V_HIP_LIB_DIR");
    let dir = std::env::var("LIGHTX2V_HIP_LIB_DIR")
        .expect("set LIGHTX2V_HIP_LIB_DIR to the directory holding liblightx2v_hip.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=lightx2v_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
}
