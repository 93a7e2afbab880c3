// The lines openmini-server's build.rs (build.rs:19-53, protobuf compilation) gains for the
// `hip-quant` cargo feature.  A build script sees the package's enabled features as
// CARGO_FEATURE_* variables (it is not compiled with them), so the check is at run time.
fn main() {
    // ... the existing tonic/prost protobuf compilation stays as it is ...
    if std::env::var_os("CARGO_FEATURE_HIP_QUANT").is_some() {
        // the directory holding libopenmini_qmm.so (openmini-v1_amd/build.py or
        // native/CMakeLists.txt of this repository)
        let dir = std::env::var("OPENMINI_QMM_DIR").expect("OPENMINI_QMM_DIR: directory of libopenmini_qmm.so");
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-lib=dylib=openmini_qmm");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
        println!("cargo:rerun-if-env-changed=OPENMINI_QMM_DIR");
    }
}
