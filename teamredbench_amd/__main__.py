from teamredbench_amd.cli import app

if __name__ == "__main__":
    app()
